/*
 * uq_layer.h -- device-resident Qwen3.5 layers of libuq.so: the per-token
 * forward of one GatedDeltaNet layer (Qwen35Forward::recr_layer,
 * crates/unltd-generation/src/qwen35_forward.rs:333-543) and of one
 * full-attention layer (attn_layer, :546-710), each with its FFN
 * (ffn, :713-768), composed from this library's quantized GEMVs and
 * per-layer ops on the caller's stream. Activations, the conv window, the
 * recurrent state and the KV cache stay in HBM; nothing is allocated and
 * nothing is copied to the host.
 *
 * Numerics are the reference forward's: every projection is
 * gemv_quant_q8k (bit-exact, uq.h), rmsnorm / l2_norm_rows / ssm_conv /
 * gdn_fused_step / the attention sums follow the reference's f32 / f64
 * steps (uq_ops.h), and the transcendentals (sigmoid, silu, softplus, the
 * gdn decay's exp, softmax's exp, swiglu, the rope angles) agree with the
 * reference's libm within 1-2 ulp. So a layer's nodes are bit-exact given
 * their inputs except where such a function enters, and a whole layer
 * agrees with the reference to the propagation of those ulps.
 */
#ifndef UQ_LAYER_H
#define UQ_LAYER_H

#include "uq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Shapes and constants of the model (Qwen35Config, crates/unltd-architectures/
 * src/qwen35.rs:252-292). The GatedDeltaNet conv has
 * channels = 2 * n_qk_heads * head_dim_linear + n_v_heads * head_dim_linear
 * (q, k, v; d_conv() = 2 * d_inner), and n_v_heads * head_dim_linear ==
 * n_embd; attention has n_head * head_dim == n_embd. */
typedef struct uq_qwen35_dims {
    size_t n_embd;          /* 4096 */
    size_t n_ff;            /* 12288 */
    size_t n_qk_heads;      /* GatedDeltaNet q/k heads (group_count): 16 */
    size_t n_v_heads;       /* GatedDeltaNet v heads: 32 */
    size_t head_dim_linear; /* 128 */
    size_t conv_kernel;     /* 4 (at most 9) */
    size_t n_head;          /* 16 */
    size_t n_head_kv;       /* 4 */
    size_t head_dim;        /* 256 (64, 128, 256 or 512) */
    size_t n_rot;           /* 64 */
    double theta_scale;     /* Qwen35Config::theta_scale() (:283-285) */
    float kq_scale;         /* Qwen35Config::kq_scale() (:277-279) */
    float rms_eps;
} uq_qwen35_dims;

/* Weights of one GatedDeltaNet layer: quantized projections as uploaded
 * handles (Q4_K or Q6_K), f32 vectors as device pointers. ssm_conv1d is the
 * GGUF tensor as stored, [channels][conv_kernel] (the forward's transpose,
 * :441-446, is folded into the conv's indexing). */
typedef struct uq_gdn_layer_w {
    uq_weights attn_qkv, attn_gate, ssm_beta, ssm_alpha, ssm_out, ffn_gate, ffn_up, ffn_down;
    const float *attn_norm;           /* [n_embd] */
    const float *ssm_dt_bias;         /* [n_v_heads] */
    const float *ssm_a;               /* [n_v_heads] */
    const float *ssm_conv1d;          /* [channels][conv_kernel] */
    const float *ssm_norm;            /* [head_dim_linear] */
    const float *post_attention_norm; /* [n_embd] */
} uq_gdn_layer_w;

/* Weights of one full-attention layer. */
typedef struct uq_attn_layer_w {
    uq_weights attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down;
    const float *attn_norm;           /* [n_embd] */
    const float *attn_q_norm;         /* [head_dim] */
    const float *attn_k_norm;         /* [head_dim] */
    const float *post_attention_norm; /* [n_embd] */
} uq_attn_layer_w;

/* Intermediate values (the reference's NodeCapture names where it has
 * them), kept in the caller's workspace after a step. */
typedef enum uq_layer_node {
    UQ_NODE_ATTN_NORM = 0, /* rmsnorm(x_in, attn_norm)                    [n_embd] */
    UQ_NODE_Z,             /* GDN: attn_gate . x                           [n_v * hd] */
    UQ_NODE_BETA_RAW,      /* GDN: ssm_beta . x                            [n_v] */
    UQ_NODE_ALPHA,         /* GDN: ssm_alpha . x                           [n_v] */
    UQ_NODE_BETA,          /* GDN: sigmoid(beta_raw)                       [n_v] */
    UQ_NODE_A_SOFTPLUS,    /* GDN: softplus(alpha + dt_bias)               [n_v] */
    UQ_NODE_GATE,          /* GDN: a_softplus * ssm_a                      [n_v] */
    UQ_NODE_CONV_RAW,      /* GDN: ssm_conv over the window                [channels] */
    UQ_NODE_CONV_SILU,     /* GDN: silu(conv_raw), its q and k parts then
                              l2-normalised in place (q/k/v_conv_predelta)  [channels] */
    UQ_NODE_GDN_OUT,       /* GDN: gdn_fused_step outputs ("attn_output")  [n_v * hd] */
    UQ_NODE_FINAL,         /* GDN: rmsnorm per head (ssm_norm) * silu(z)   [n_v * hd] */
    UQ_NODE_QFULL,         /* attention: attn_q . x, per head q | gate      [2 * n_head * head_dim] */
    UQ_NODE_K_RAW,         /* attention: attn_k . x                        [n_head_kv * head_dim] */
    UQ_NODE_Q,             /* attention: q normed and rotated              [n_head * head_dim] */
    UQ_NODE_ATTN,          /* attention: softmax(q K^T) V per head         [n_head * head_dim] */
    UQ_NODE_GATED,         /* attention: attn * sigmoid(gate)              [n_head * head_dim] */
    UQ_NODE_ATTN_OUT,      /* ssm_out / attn_output projection ("linear_attn_out") [n_embd] */
    UQ_NODE_RESIDUAL,      /* x_in + attn_out                              [n_embd] */
    UQ_NODE_POST_NORM,     /* rmsnorm(residual, post_attention_norm)       [n_embd] */
    UQ_NODE_FFN_GATE,      /* ffn_gate . p                                 [n_ff] */
    UQ_NODE_FFN_UP,        /* ffn_up . p                                   [n_ff] */
    UQ_NODE_FFN_SWIGLU,    /* swiglu(gate, up)                             [n_ff] */
    UQ_NODE_FFN_OUT,       /* ffn_down . swiglu                            [n_embd] */
    UQ_NODE_SOFT,          /* attention: softmax weights [n_head][pos + 1], room for
                              [n_head][n_ctx_max] (last: the other nodes' offsets
                              do not depend on n_ctx_max)                  */
    UQ_NODE_COUNT
} uq_layer_node;

/* Workspace of a layer step in floats (both layer kinds; n_ctx_max sizes
 * the attention's softmax rows, 0 for a GatedDeltaNet layer), and where a
 * node sits in it. */
size_t uq_layer_ws_floats(const uq_qwen35_dims *d, size_t n_ctx_max);
uq_status uq_layer_node_at(const uq_qwen35_dims *d, size_t n_ctx_max, int node, size_t *offset, size_t *count);

/* One token through a GatedDeltaNet layer (recr_layer): l_out = residual +
 * ffn(residual), residual = x_in + ssm_out(final). State, carried from token
 * to token by the caller:
 *   d_conv_win [conv_kernel][channels]: rows 0..conv_kernel-2 are the
 *     reference's conv ring (zeros before the first token); the step writes
 *     the token's qkv projection into the last row, convolves, then shifts
 *     the rows up (:449-450), so after the step the last two rows both hold
 *     this token's qkv ("linear_attn_qkv_mixed");
 *   d_state [n_v_heads][head_dim_linear][head_dim_linear]: the recurrent
 *     state, S[i][j] at i * hd + j (zeros before the first token).
 * d_x_in and d_l_out may not overlap the workspace or the state.
 * Errors: UQ_ERR_ARG (bad dims, handle, pointer or a workspace below
 * uq_layer_ws_floats), UQ_ERR_LEN (a projection's shape does not match the
 * dims), UQ_ERR_DTYPE (a projection that is not Q4_K / Q6_K). */
uq_status uq_gdn_layer_step_d(const uq_qwen35_dims *d, const uq_gdn_layer_w *w, float *d_conv_win, float *d_state,
                              const float *d_x_in, float *d_l_out, float *d_ws, size_t ws_floats, void *stream);

/* One token at position pos through a full-attention layer (attn_layer).
 * The caches hold rows [p][n_head_kv][head_dim] for p < n_ctx_max (the
 * reference's k_cache / v_cache slots, :644-645); the step writes row pos
 * (k normed and rotated, v as projected) and attends over rows 0..pos.
 * pos >= n_ctx_max is UQ_ERR_ARG (the reference's "context full"
 * refusal, :298-303); other errors as uq_gdn_layer_step_d. */
uq_status uq_attn_layer_step_d(const uq_qwen35_dims *d, const uq_attn_layer_w *w, float *d_k_cache,
                               float *d_v_cache, size_t n_ctx_max, size_t pos, const float *d_x_in, float *d_l_out,
                               float *d_ws, size_t ws_floats, void *stream);

/* Prefill: n_tokens tokens through a layer in one call, with the same
 * results as n_tokens successive step calls, bit for bit (layer outputs,
 * conv window, recurrent state, KV cache rows). The reference prefills token
 * by token (crates/unltd-generation/src/greedy.rs:55-65); here every
 * projection of the layer runs once over all the tokens as uq_gemm_q8k (each
 * row equals the token's gemv_quant_q8k, quants.rs:474-515), the norms and
 * the FFN's swiglu and residual adds over all the rows, and the recurrent
 * part (conv, norms, gates, gdn_fused_step, gated norm) or the attention
 * core (q / k norms, IMROPE, causal attention) token after token, since
 * token t depends on tokens before it there: the recurrent part in one
 * launch over all the tokens for head_dim_linear 64 or 128 (else with the
 * step's launches per token), the attention core with the step's launches.
 * d_x_in and d_l_out are [n_tokens][n_embd]. The workspace
 * (uq_layer_prefill_ws_floats; 256-byte aligned, as hipMalloc returns) holds
 * the step's node space (its contents after the call unspecified), n_tokens
 * rows of each batched value and the q8k GEMM's workspace: nothing is
 * allocated. n_tokens == 0 is a no-op.
 * uq_layer_prefill_ws_floats takes the layer's weights (either kind, or
 * both for a workspace shared by the two; the other may be NULL) and
 * returns 0 for bad dims or n_tokens == 0. */
size_t uq_layer_prefill_ws_floats(const uq_qwen35_dims *d, const uq_gdn_layer_w *gdn, const uq_attn_layer_w *attn,
                                  size_t n_ctx_max, size_t n_tokens);

/* n_tokens successive uq_gdn_layer_step_d calls (recr_layer,
 * qwen35_forward.rs:333-543): tokens t = 0 .. n_tokens - 1 of d_x_in, the
 * window and state carried through them as the step carries them. Errors as
 * uq_gdn_layer_step_d. */
uq_status uq_gdn_layer_prefill_d(const uq_qwen35_dims *d, const uq_gdn_layer_w *w, float *d_conv_win, float *d_state,
                                 size_t n_tokens, const float *d_x_in, float *d_l_out, float *d_ws, size_t ws_floats,
                                 void *stream);

/* n_tokens successive uq_attn_layer_step_d calls (attn_layer, :546-710) at
 * positions pos0 .. pos0 + n_tokens - 1: their cache rows are written and
 * token t attends over rows 0 .. pos0 + t. A last position at or beyond
 * n_ctx_max is UQ_ERR_ARG (the reference's "context full", :298-303);
 * other errors as uq_attn_layer_step_d. */
uq_status uq_attn_layer_prefill_d(const uq_qwen35_dims *d, const uq_attn_layer_w *w, float *d_k_cache,
                                  float *d_v_cache, size_t n_ctx_max, size_t pos0, size_t n_tokens,
                                  const float *d_x_in, float *d_l_out, float *d_ws, size_t ws_floats, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* UQ_LAYER_H */
