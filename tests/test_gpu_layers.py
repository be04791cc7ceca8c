"""GPU parity of the device-resident layers (include/uq_layer.h) against the
oracle's restatement of Qwen35Forward::recr_layer / attn_layer / ffn
(qwen35_forward.rs:333-768, oracle.recr_layer / attn_layer).

Two checks per layer kind:
  * stage by stage: every node of the device step is recomputed by the
    oracle from the device's own inputs to that stage. Bit-exact where the
    reference's arithmetic has no libm call (rmsnorm, the q8k projections,
    ssm_conv, the f32 products and sums, the residuals); within the stated
    ulps where the device's correctly rounded exp / log / sin / cos meet the
    C library's (sigmoid, softplus, silu, swiglu 2 ulp; the gdn decay and
    softmax 2 ulp; the rope rotation 1 ulp), as tests/test_gpu_ops.py bounds
    each op alone;
  * whole tokens: several tokens (recurrent state and conv window carried,
    KV cache growing) against the oracle run from the same inputs. Those
    ulps then pass through the Q8_K quantization of the next projection's
    input, where one may move an element across a rounding boundary, so the
    bar is |dev - ref| <= 1e-3 * (|ref| + rms(ref)) per element.
Shapes: a small model (n_embd 512) for several tokens, and the 9B shapes of
the decode benchmark (n_embd 4096, n_ff 12288, 16/32 GatedDeltaNet heads of
128, attention 16/4 heads of 256) for one GatedDeltaNet and two attention
tokens.
"""
import os
import sys
import types

import numpy as np
import pytest

import oracle as O
import uq
import uq.synth as S
from uq import layer as L

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)

SMALL = dict(n_embd=512, n_ff=1024, n_qk_heads=4, n_v_heads=8, head_dim_linear=64, conv_kernel=4, n_head=4,
             n_head_kv=2, head_dim=128, n_rot=32)
FULL = dict(n_embd=4096, n_ff=12288, n_qk_heads=16, n_v_heads=32, head_dim_linear=128, conv_kernel=4, n_head=16,
            n_head_kv=4, head_dim=256, n_rot=64)


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dims(shape):
    # theta_scale = freq_base^(-2/n_rot) in f32 (qwen35.rs:283-285), kq_scale = 1/sqrt(head_dim)
    theta = float(np.float32(1.0e7) ** np.float32(-2.0 / shape["n_rot"]))
    kq = float(np.float32(1.0) / np.sqrt(np.float32(shape["head_dim"])))
    d = L.Dims(**shape, theta_scale=theta, kq_scale=kq, rms_eps=1e-6)
    cfg = types.SimpleNamespace(**shape, theta_scale=theta, kq_scale=kq, rms_eps=np.float32(1e-6))
    return d, cfg


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)


def assert_bitwise(got, ref, what):
    bad = np.nonzero(bits(got) != bits(ref))[0]
    assert bad.size == 0, f"{what}: {bad.size} of {len(bits(ref))} differ, first {bad[:5].tolist()}"


def assert_ulp(got, ref, max_ulp, what):
    d = np.abs(bits(got) - bits(ref))
    assert d.max() <= max_ulp, f"{what}: {int(d.max())} ulp at {int(np.argmax(d))}"


def assert_token(got, ref, what):
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    err = np.abs(got.astype(np.float64) - ref)
    bad = np.nonzero(err > 1e-3 * (np.abs(ref) + rms))[0]
    assert bad.size == 0, f"{what}: {bad.size} outside, worst {float(err.max()):.3g} (rms {rms:.3g})"
    log(f"{what}: max |dev - ref| = {float(err.max()):.3g}, {int(np.sum(err == 0))}/{err.size} equal")


def vec(rng, n, kind):
    if kind == "norm":
        return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    if kind == "a":  # ssm_a = -exp(A_log) < 0: exp(gate) decays the state
        return (-np.exp(0.5 * rng.standard_normal(n))).astype(np.float32)
    return (kind * rng.standard_normal(n)).astype(np.float32)


class Model:
    """Random weights of one layer of each kind, on host and device."""

    def __init__(self, shape, seed, q6=False):
        self.d, self.cfg = dims(shape)
        c = self.cfg
        n, nff, nv, hd = c.n_embd, c.n_ff, c.n_v_heads, c.head_dim_linear
        ch = self.d.channels
        rng = np.random.default_rng(seed)
        dt = S.Q6_K if q6 else S.Q4_K  # attn_qkv, ffn_down, attn_v: Q4_K or Q6_K (qwen35_forward.rs:167-201)
        gproj = {"attn_qkv": (n, ch, dt), "attn_gate": (n, nv * hd, S.Q4_K), "ssm_beta": (n, nv, S.Q4_K),
                 "ssm_alpha": (n, nv, S.Q4_K), "ssm_out": (nv * hd, n, S.Q4_K), "ffn_gate": (n, nff, S.Q4_K),
                 "ffn_up": (n, nff, S.Q4_K), "ffn_down": (nff, n, dt)}
        aproj = {"attn_q": (n, 2 * c.n_head * c.head_dim, S.Q4_K), "attn_k": (n, c.n_head_kv * c.head_dim, S.Q4_K),
                 "attn_v": (n, c.n_head_kv * c.head_dim, dt), "attn_output": (c.n_head * c.head_dim, n, S.Q4_K),
                 "ffn_gate": (n, nff, S.Q4_K), "ffn_up": (n, nff, S.Q4_K), "ffn_down": (nff, n, dt)}
        gvec = {"attn_norm": (n, "norm"), "ssm_dt_bias": (nv, 1.0), "ssm_a": (nv, "a"),
                "ssm_conv1d": (ch * c.conv_kernel, 0.3), "ssm_norm": (hd, "norm"), "post_attention_norm": (n, "norm")}
        avec = {"attn_norm": (n, "norm"), "attn_q_norm": (c.head_dim, "norm"), "attn_k_norm": (c.head_dim, "norm"),
                "post_attention_norm": (n, "norm")}
        self.dev = []

        def build(proj, vecs, salt):
            host, devw = {}, {}
            for i, (name, (K, N, t)) in enumerate(proj.items()):
                # block scales sized so that a projection keeps activations near unit scale
                sigma = 1.0 / ((300.0 if t == S.Q4_K else 500.0) * np.sqrt(K))
                b = S.weights(t, N, K, seed=seed * 1000 + salt + i, sigma=sigma)
                host[name] = (b, t)
                devw[name] = uq.Weights(b, t, K, N)
            for name, (m, kind) in vecs.items():
                host[name] = vec(rng, m, kind)
                devw[name] = uq.DeviceArray.from_numpy(host[name])
            self.dev += list(devw.values())
            return host, devw

        self.gh, gd = build(gproj, gvec, 0)
        self.ah, ad = build(aproj, avec, 500)
        self.gw, self.aw = L.GdnWeights(**gd), L.AttnWeights(**ad)

    def free(self):
        for o in self.dev:
            o.free()


def nodes_of(d, ws, names, n_ctx_max=0):
    full = ws.download(np.float32, ws.nbytes // 4)
    out = {}
    for nm in names:
        off, cnt = L.node_at(d, nm, n_ctx_max)
        out[nm] = full[off:off + cnt].copy()
    return out


def q8k(w, x, dim_in, dim_out):
    out = np.zeros(dim_out, np.float32)
    O.gemv_quant_q8k(out, x, w[0], dim_in, dim_out, w[1], nthreads=NT)
    return out


def check_ffn_stages(cfg, host, D, x_in, l_out, what):
    """post_attention_norm, the q8k FFN and the residuals, from the device's nodes."""
    n, nff = cfg.n_embd, cfg.n_ff
    assert_bitwise(D["residual"], x_in + D["attn_out"], f"{what} residual")
    assert_bitwise(D["post_norm"], O.rmsnorm(D["residual"], host["post_attention_norm"], cfg.rms_eps),
                   f"{what} post_norm")
    assert_bitwise(D["ffn_gate"], q8k(host["ffn_gate"], D["post_norm"], n, nff), f"{what} ffn_gate")
    assert_bitwise(D["ffn_up"], q8k(host["ffn_up"], D["post_norm"], n, nff), f"{what} ffn_up")
    assert_ulp(D["ffn_swiglu"], O.swiglu(D["ffn_gate"], D["ffn_up"]), 2, f"{what} ffn_swiglu")
    assert_bitwise(D["ffn_out"], q8k(host["ffn_down"], D["ffn_swiglu"], nff, n), f"{what} ffn_out")
    assert_bitwise(l_out, D["residual"] + D["ffn_out"], f"{what} l_out")


GDN_NODES = ["attn_norm", "z", "beta_raw", "alpha", "beta", "a_softplus", "gate", "conv_raw", "conv_silu", "gdn_out",
             "final", "attn_out", "residual", "post_norm", "ffn_gate", "ffn_up", "ffn_swiglu", "ffn_out"]
ATTN_NODES = ["attn_norm", "qfull", "k_raw", "q", "attn", "gated", "attn_out", "residual", "post_norm", "ffn_gate",
              "ffn_up", "ffn_swiglu", "ffn_out", "soft"]


def run_gdn(m, ntok, seed):
    d, c, h = m.d, m.cfg, m.gh
    n, nqk, nv, hd, ck = c.n_embd, c.n_qk_heads, c.n_v_heads, c.head_dim_linear, c.conv_kernel
    ch = d.channels
    win = uq.DeviceArray.from_numpy(np.zeros(ck * ch, np.float32))
    state = uq.DeviceArray.from_numpy(np.zeros(nv * hd * hd, np.float32))
    ws = uq.DeviceArray(4 * L.ws_floats(d))
    dl = uq.DeviceArray(4 * n)
    ring, st = np.zeros((ck - 1, ch), np.float32), np.zeros((nv, hd, hd), np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    for t in range(ntok):
        x = S.activations(n, seed=seed + t)
        pre_win = win.download(np.float32, ck * ch).reshape(ck, ch)
        pre_state = state.download(np.float32, nv * hd * hd).reshape(nv, hd, hd)
        dx = uq.DeviceArray.from_numpy(x)
        L.gdn_step(d, m.gw, win, state, dx, dl, ws)
        got = dl.download(np.float32, n)
        D = nodes_of(d, ws, GDN_NODES)
        post_win = win.download(np.float32, ck * ch).reshape(ck, ch)
        what = f"gdn n_embd={n} token {t}"
        log(what)
        # --- stage by stage, from the device's own inputs
        assert_bitwise(D["attn_norm"], O.rmsnorm(x, h["attn_norm"], c.rms_eps), f"{what} attn_norm")
        qkv = post_win[-1]
        assert_bitwise(qkv, q8k(h["attn_qkv"], D["attn_norm"], n, ch), f"{what} qkv")
        assert_bitwise(post_win[:-1], np.concatenate([pre_win[1:-1], qkv[None]]), f"{what} ring shift")
        assert_bitwise(D["z"], q8k(h["attn_gate"], D["attn_norm"], n, nv * hd), f"{what} z")
        assert_bitwise(D["beta_raw"], q8k(h["ssm_beta"], D["attn_norm"], n, nv), f"{what} beta_raw")
        assert_bitwise(D["alpha"], q8k(h["ssm_alpha"], D["attn_norm"], n, nv), f"{what} alpha")
        assert_ulp(D["beta"], O.sigmoid(D["beta_raw"]), 2, f"{what} beta")
        assert_ulp(D["a_softplus"], O.softplus(D["alpha"] + h["ssm_dt_bias"]), 2, f"{what} a_softplus")
        assert_bitwise(D["gate"], D["a_softplus"] * h["ssm_a"], f"{what} gate")
        kern = np.ascontiguousarray(h["ssm_conv1d"].reshape(ch, ck).T).reshape(-1)
        win_in = np.concatenate([pre_win[:-1].reshape(-1), qkv])
        assert_bitwise(D["conv_raw"], O.ssm_conv(win_in, kern, ck, ch), f"{what} conv_raw")
        mix = O.silu(D["conv_raw"])
        assert_ulp(D["conv_silu"][2 * nqk * hd:], mix[2 * nqk * hd:], 2, f"{what} v_conv")
        assert_ulp(D["conv_silu"][:2 * nqk * hd], O.l2_norm_rows(mix[:2 * nqk * hd], hd, c.rms_eps), 4,
                   f"{what} q/k_conv")
        qc, kc, vc = (D["conv_silu"][:nqk * hd], D["conv_silu"][nqk * hd:2 * nqk * hd], D["conv_silu"][2 * nqk * hd:])
        new_state = state.download(np.float32, nv * hd * hd).reshape(nv, hd, hd)
        for hh in range(nv):
            qk = hh % nqk
            s_ref, o_ref = O.gdn_fused_step(pre_state[hh].reshape(-1), qc[qk * hd:(qk + 1) * hd],
                                            kc[qk * hd:(qk + 1) * hd], vc[hh * hd:(hh + 1) * hd], float(D["gate"][hh]),
                                            float(D["beta"][hh]), float(scale))
            assert_ulp(D["gdn_out"][hh * hd:(hh + 1) * hd], o_ref, 4, f"{what} gdn_out head {hh}")
            assert_ulp(new_state[hh].reshape(-1), s_ref, 4, f"{what} state head {hh}")
        normed = np.concatenate([O.rmsnorm(D["gdn_out"][i * hd:(i + 1) * hd], h["ssm_norm"], c.rms_eps)
                                 for i in range(nv)])
        assert_ulp(D["final"], normed * O.silu(D["z"]), 3, f"{what} final")
        assert_bitwise(D["attn_out"], q8k(h["ssm_out"], D["final"], nv * hd, n), f"{what} attn_out")
        check_ffn_stages(c, h, D, x, got, what)
        # --- the whole token against the oracle's layer run from the same inputs
        ref, _ = O.recr_layer(c, h, ring, st, x, nthreads=NT)
        assert_token(got, ref, f"{what} l_out vs oracle recr_layer")
        dx.free()
    for a in (win, state, ws, dl):
        a.free()


def run_attn(m, ntok, n_ctx_max, seed):
    d, c, h = m.d, m.cfg, m.ah
    n, nh, nkv, hd = c.n_embd, c.n_head, c.n_head_kv, c.head_dim
    kv = nkv * hd
    kc = uq.DeviceArray.from_numpy(np.zeros(n_ctx_max * kv, np.float32))
    vcache = uq.DeviceArray.from_numpy(np.zeros(n_ctx_max * kv, np.float32))
    ws = uq.DeviceArray(4 * L.ws_floats(d, n_ctx_max))
    dl = uq.DeviceArray(4 * n)
    kref, vref = np.zeros((n_ctx_max, kv), np.float32), np.zeros((n_ctx_max, kv), np.float32)
    for pos in range(ntok):
        x = S.activations(n, seed=seed + pos)
        dx = uq.DeviceArray.from_numpy(x)
        L.attn_step(d, m.aw, kc, vcache, n_ctx_max, pos, dx, dl, ws)
        got = dl.download(np.float32, n)
        D = nodes_of(d, ws, ATTN_NODES, n_ctx_max)
        K = kc.download(np.float32, n_ctx_max * kv).reshape(n_ctx_max, kv)
        V = vcache.download(np.float32, n_ctx_max * kv).reshape(n_ctx_max, kv)
        what = f"attn n_embd={n} pos {pos}"
        log(what)
        assert_bitwise(D["attn_norm"], O.rmsnorm(x, h["attn_norm"], c.rms_eps), f"{what} attn_norm")
        assert_bitwise(D["qfull"], q8k(h["attn_q"], D["attn_norm"], n, 2 * nh * hd), f"{what} qfull")
        assert_bitwise(D["k_raw"], q8k(h["attn_k"], D["attn_norm"], n, kv), f"{what} k_raw")
        assert_bitwise(V[pos], q8k(h["attn_v"], D["attn_norm"], n, kv), f"{what} v row")
        qn = [O.rmsnorm(D["qfull"][2 * i * hd:2 * i * hd + hd], h["attn_q_norm"], c.rms_eps) for i in range(nh)]
        assert_ulp(D["q"], np.concatenate([O.rope_imrope(q, c.n_rot, c.theta_scale, pos) for q in qn]), 1,
                   f"{what} q")
        kn = [O.rmsnorm(D["k_raw"][i * hd:(i + 1) * hd], h["attn_k_norm"], c.rms_eps) for i in range(nkv)]
        assert_ulp(K[pos], np.concatenate([O.rope_imrope(k, c.n_rot, c.theta_scale, pos) for k in kn]), 1,
                   f"{what} k row")
        a_ref, s_ref = O.attn_decode(D["q"], K[:pos + 1], V[:pos + 1], pos + 1, nh, nkv, hd, c.kq_scale)
        assert_ulp(D["soft"][:nh * (pos + 1)], s_ref, 2, f"{what} soft")
        assert_ulp(D["attn"], a_ref, 2, f"{what} attn")
        gate = np.concatenate([D["qfull"][2 * i * hd + hd:2 * (i + 1) * hd] for i in range(nh)])
        assert_ulp(D["gated"], D["attn"] * O.sigmoid(gate), 2, f"{what} gated")
        assert_bitwise(D["attn_out"], q8k(h["attn_output"], D["gated"], nh * hd, n), f"{what} attn_out")
        check_ffn_stages(c, h, D, x, got, what)
        ref, _ = O.attn_layer(c, h, kref, vref, pos, x, nthreads=NT)
        assert_token(got, ref, f"{what} l_out vs oracle attn_layer")
        dx.free()
    for a in (kc, vcache, ws, dl):
        a.free()


@pytest.mark.parametrize("q6", [False, True])
def test_gdn_layer_small(q6):
    m = Model(SMALL, seed=11 + q6, q6=q6)
    try:
        run_gdn(m, ntok=4, seed=100)
    finally:
        m.free()


@pytest.mark.parametrize("q6", [False, True])
def test_attn_layer_small(q6):
    m = Model(SMALL, seed=21 + q6, q6=q6)
    try:
        run_attn(m, ntok=5, n_ctx_max=8, seed=200)
    finally:
        m.free()


def test_gdn_layer_wide_heads():
    """GatedDeltaNet heads of 2048 (one q/k head, two v heads): above the
    1024 of the one-launch conv / l2-norm / gates kernel and the 128 of the
    register-resident delta rule, so the step runs the separate glue launches
    and the workgroup-per-head delta rule; the same bar as every layer."""
    wide = dict(SMALL, n_embd=4096, n_qk_heads=1, n_v_heads=2, head_dim_linear=2048, n_head=16, n_head_kv=4,
                head_dim=256, n_rot=64)
    m = Model(wide, seed=61)
    try:
        run_gdn(m, ntok=2, seed=600)
    finally:
        m.free()


def test_layers_wide_embedding():
    """n_embd 5120: the projections of a norm take the two-task streaming
    kernel, which does not form the norm in its prologue, so the steps run
    the norm launches (attn_norm; residual + post_attention_norm) before them."""
    wide = dict(SMALL, n_embd=5120, n_qk_heads=10, n_v_heads=40, head_dim_linear=128, n_head=20, n_head_kv=5,
                head_dim=256, n_rot=64)
    m = Model(wide, seed=71)
    try:
        run_gdn(m, ntok=1, seed=700)
        run_attn(m, ntok=2, n_ctx_max=4, seed=800)
    finally:
        m.free()


def test_layers_9b_shapes():
    """The decode benchmark's layer shapes (Q6_K on the attention layer's
    v and down projections, as its every-4th-layer mix)."""
    m = Model(FULL, seed=31, q6=True)
    try:
        run_gdn(m, ntok=1, seed=300)
        run_attn(m, ntok=2, n_ctx_max=4, seed=400)
    finally:
        m.free()


def test_layer_step_refuses_context_full():
    m = Model(SMALL, seed=41)
    try:
        d = m.d
        kc, vc = uq.DeviceArray(4 * 2 * 256), uq.DeviceArray(4 * 2 * 256)
        ws, dx, dl = uq.DeviceArray(4 * L.ws_floats(d, 2)), uq.DeviceArray(4 * 512), uq.DeviceArray(4 * 512)
        with pytest.raises(uq.UqError) as e:
            L.attn_step(d, m.aw, kc, vc, 2, 2, dx, dl, ws)
        assert e.value.kind == "ARG" and "context full" in str(e.value)
        for a in (kc, vc, ws, dx, dl):
            a.free()
    finally:
        m.free()


def test_layer_steps_replay_in_a_graph():
    """Both steps captured in one HIP graph (they allocate nothing and hold
    no memset): every replay from the same saved state gives the eager run's
    bits, with eager work and synchronisations between the replays."""
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(__file__))))
    import bench
    m = Model(SMALL, seed=51, q6=True)
    hip = bench.Hip()
    s = hip.stream()
    try:
        d, c = m.d, m.cfg
        n, ch, ctx = c.n_embd, d.channels, 8
        win0 = (0.5 * np.random.default_rng(1).standard_normal(c.conv_kernel * ch)).astype(np.float32)
        st0 = np.zeros(c.n_v_heads * c.head_dim_linear ** 2, np.float32)
        kv = c.n_head_kv * c.head_dim
        k0 = np.random.default_rng(2).standard_normal(ctx * kv).astype(np.float32) / 16
        v0 = np.random.default_rng(3).standard_normal(ctx * kv).astype(np.float32)
        win, state = uq.DeviceArray.from_numpy(win0), uq.DeviceArray.from_numpy(st0)
        kc, vc = uq.DeviceArray.from_numpy(k0), uq.DeviceArray.from_numpy(v0)
        ws = uq.DeviceArray(4 * L.ws_floats(d, ctx))
        dx = uq.DeviceArray.from_numpy(S.activations(n, seed=7))
        y1, y2 = uq.DeviceArray(4 * n), uq.DeviceArray(4 * n)

        def reset():
            win.upload(win0)
            state.upload(st0)
            kc.upload(k0)
            vc.upload(v0)
            hip.sync()

        def steps():
            L.gdn_step(d, m.gw, win, state, dx, y1, ws, s)
            L.attn_step(d, m.aw, kc, vc, ctx, 5, y1, y2, ws, s)

        reset()
        steps()
        hip.sync()
        ref = (y2.download(np.float32, n), state.download(np.float32, st0.size), kc.download(np.float32, k0.size))
        reset()
        g = hip.capture(s, steps)
        for r in range(3):
            reset()
            y2.upload(np.zeros(n, np.float32))
            hip.launch_graph(g, s)
            hip.sync()
            got = (y2.download(np.float32, n), state.download(np.float32, st0.size), kc.download(np.float32, k0.size))
            for a, b, what in zip(got, ref, ("l_out", "gdn state", "k cache")):
                assert_bitwise(a, b, f"replay {r} {what}")
        for a in (win, state, kc, vc, ws, dx, y1, y2):
            a.free()
    finally:
        m.free()
