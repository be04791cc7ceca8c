"""The oracle's layer restatement (oracle.recr_layer / attn_layer, after
qwen35_forward.rs:333-768) pinned where the mathematics fixes the answer,
so that a wrong slice, head mapping or step order fails here before it is
used to judge the device:

  * GatedDeltaNet, first token (conv ring and state zero): the conv of the
    window [0, 0, 0, qkv] is the last kernel tap times qkv, exactly; the
    delta rule from S = 0 gives d = v * beta and S = k d^T, so each v head's
    output is d_j * (k . q) * scale of its q/k head h % n_qk;
  * second token: the ring holds the first token's qkv in its last row, so
    the conv is the f32 sum of the last two taps;
  * attention at position 0: the softmax over one position is 1, so each q
    head's attention output is its kv head's (h / group) value row exactly,
    and the gated output is that row times sigmoid of the head's gate half;
  * a layer whose projections are all zero returns its input.
"""
import types

import numpy as np

import oracle as O
import uq.synth as S

SHAPE = dict(n_embd=256, n_ff=512, n_qk_heads=2, n_v_heads=4, head_dim_linear=64, conv_kernel=4, n_head=2,
             n_head_kv=1, head_dim=128, n_rot=32)


def cfg():
    return types.SimpleNamespace(**SHAPE, theta_scale=0.5, kq_scale=float(1 / np.sqrt(128.0)),
                                 rms_eps=np.float32(1e-6))


def weights(seed, zero=False):
    c = cfg()
    n, nff, nv, hd = c.n_embd, c.n_ff, c.n_v_heads, c.head_dim_linear
    ch = 2 * c.n_qk_heads * hd + nv * hd
    rng = np.random.default_rng(seed)
    shapes = {"attn_qkv": (n, ch), "attn_gate": (n, nv * hd), "ssm_beta": (n, nv), "ssm_alpha": (n, nv),
              "ssm_out": (nv * hd, n), "ffn_gate": (n, nff), "ffn_up": (n, nff), "ffn_down": (nff, n),
              "attn_q": (n, 2 * c.n_head * c.head_dim), "attn_k": (n, c.n_head_kv * c.head_dim),
              "attn_v": (n, c.n_head_kv * c.head_dim), "attn_output": (c.n_head * c.head_dim, n)}
    w = {}
    for i, (name, (K, N)) in enumerate(shapes.items()):
        b = S.weights(S.Q4_K, N, K, seed=seed * 100 + i, sigma=1.0 / (300 * np.sqrt(K)))
        if zero:
            b = np.zeros_like(b)
        w[name] = (b, S.Q4_K)
    f = lambda m, s=1.0: (s * rng.standard_normal(m)).astype(np.float32)
    w.update(attn_norm=1 + f(n, 0.1), ssm_dt_bias=f(nv), ssm_a=-np.exp(f(nv, 0.5)), ssm_conv1d=f(ch * 4, 0.3),
             ssm_norm=1 + f(hd, 0.1), post_attention_norm=1 + f(n, 0.1), attn_q_norm=1 + f(c.head_dim, 0.1),
             attn_k_norm=1 + f(c.head_dim, 0.1))
    return w, ch


def test_recr_layer_first_tokens_closed_forms():
    c = cfg()
    w, ch = weights(1)
    nqk, nv, hd, ck = c.n_qk_heads, c.n_v_heads, c.head_dim_linear, c.conv_kernel
    ring, st = np.zeros((ck - 1, ch), np.float32), np.zeros((nv, hd, hd), np.float32)
    x0 = S.activations(c.n_embd, seed=3)
    _, nd = O.recr_layer(c, w, ring, st, x0)
    kern = w["ssm_conv1d"].reshape(ch, ck)
    assert np.array_equal(nd["conv_raw"], nd["qkv"] * kern[:, 3]), "first-token conv is the last tap"
    assert np.array_equal(ring[-1], nd["qkv"]) and not ring[:-1].any(), "ring holds the token's qkv last"
    qc, kc, vc = (nd["conv_silu"][:nqk * hd], nd["conv_silu"][nqk * hd:2 * nqk * hd], nd["conv_silu"][2 * nqk * hd:])
    scale = 1.0 / np.sqrt(hd)
    for h in range(nv):
        qk = h % nqk
        d = vc[h * hd:(h + 1) * hd].astype(np.float64) * nd["beta"][h]
        kq = float(np.dot(kc[qk * hd:(qk + 1) * hd].astype(np.float64), qc[qk * hd:(qk + 1) * hd]))
        np.testing.assert_allclose(nd["gdn_out"][h * hd:(h + 1) * hd], d * kq * scale, rtol=2e-5, atol=1e-7,
                                   err_msg=f"v head {h} (q/k head {qk})")
        np.testing.assert_allclose(st[h], np.outer(kc[qk * hd:(qk + 1) * hd], d), rtol=1e-6, atol=1e-9)
    q0 = nd["qkv"]
    x1 = S.activations(c.n_embd, seed=4)
    _, nd1 = O.recr_layer(c, w, ring, st, x1)
    expect = (q0 * kern[:, 2]) + (nd1["qkv"] * kern[:, 3])  # 0 + 0 + a + b, f32
    assert np.array_equal(nd1["conv_raw"], expect.astype(np.float32)), "second-token conv"


def test_attn_layer_position_zero_closed_forms():
    c = cfg()
    w, _ = weights(2)
    nh, nkv, hd = c.n_head, c.n_head_kv, c.head_dim
    kc, vc = np.zeros((4, nkv * hd), np.float32), np.zeros((4, nkv * hd), np.float32)
    x = S.activations(c.n_embd, seed=5)
    _, nd = O.attn_layer(c, w, kc, vc, 0, x)
    assert np.all(nd["soft"] == 1.0)
    group = nh // nkv
    for h in range(nh):
        v = vc[0, (h // group) * hd:(h // group + 1) * hd]
        assert np.array_equal(nd["attn"][h * hd:(h + 1) * hd], v), f"head {h} takes kv head {h // group}"
        gate = nd["qfull"][2 * h * hd + hd:2 * (h + 1) * hd]
        assert np.array_equal(nd["gated"][h * hd:(h + 1) * hd], v * O.sigmoid(gate)), f"head {h} gate half"
    assert np.array_equal(kc[0], nd["k_row"]) and np.array_equal(vc[0], nd["v_row"])


def test_zero_projections_return_the_input():
    c = cfg()
    w, ch = weights(3, zero=True)
    x = S.activations(c.n_embd, seed=6)
    ring, st = np.zeros((c.conv_kernel - 1, ch), np.float32), np.zeros((c.n_v_heads, 64, 64), np.float32)
    l, _ = O.recr_layer(c, w, ring, st, x)
    assert np.array_equal(l, x)
    kc, vc = np.zeros((2, c.n_head_kv * c.head_dim), np.float32), np.zeros((2, c.n_head_kv * c.head_dim), np.float32)
    l, _ = O.attn_layer(c, w, kc, vc, 1, x)
    assert np.array_equal(l, x)
