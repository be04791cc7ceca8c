"""The oracle's per-layer ops (oracle/oracle_ops.c) against the reference's
own tests of crates/unltd-tensor/src/kernels.rs (each test below restates
one, cited by line) and against independent restatements in Python for
inputs those tests leave open (sequential and pairwise f64 sums written out
as loops, the rope angle recursion, the gdn column chain)."""
import ctypes
import math

import numpy as np
import pytest

import oracle as O

f32 = np.float32
_libm = ctypes.CDLL("libm.so.6")
_libm.expf.argtypes = [ctypes.c_float]
_libm.expf.restype = ctypes.c_float
_libm.fma.argtypes = [ctypes.c_double] * 3
_libm.fma.restype = ctypes.c_double


def expf(v):
    """The C library's expf, which Rust's f32::exp calls (numpy's float32 exp
    is a different implementation)."""
    return f32(_libm.expf(float(v)))


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_rmsnorm_exact_cases():  # kernels.rs:449-487
    assert (O.rmsnorm([1.0] * 4, [1.0] * 4, 0.0) == 1.0).all()
    out = O.rmsnorm([3.0, 4.0], [1.0, 1.0], 0.0)
    mean = f32((9.0 + 16.0) / 2.0)
    scale = f32(1.0) / np.sqrt(mean + f32(0.0))
    assert bits(out).tolist() == bits([f32(3.0) * scale, f32(4.0) * scale]).tolist()
    assert (O.rmsnorm([0.0, 0.0], [2.0, 3.0], 1e-6) == 0.0).all()
    x = np.full(4, 1e8, np.float32)
    sq = f32(1e8) * f32(1e8)
    assert float(sq) != 1e16
    scale = f32(1.0) / np.sqrt(sq + f32(0.0))
    assert bits(O.rmsnorm(x, np.ones(4, np.float32), 0.0)).tolist() == bits(x * scale).tolist()


def _rmsnorm_py(x, w, eps):
    s = 0.0
    for v in x:
        s += float(f32(v) * f32(v))  # f32 square, sequential f64 sum
    mean = f32(s / len(x))
    scale = f32(1.0) / np.sqrt(f32(mean + f32(eps)))
    return (x * scale) * w


def test_rmsnorm_matches_sequential_restatement():
    rng = np.random.default_rng(1)
    for n in (1, 7, 256, 4096):
        x = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 30.0])).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        assert bits(O.rmsnorm(x, w, 1e-6)).tolist() == bits(_rmsnorm_py(x, w, 1e-6)).tolist()


def test_l2_norm_rows_reference_formula():  # kernels.rs:663-693
    assert O.l2_norm_rows([3.0, 4.0], 2, 1e-6).tolist() == [f32(0.6), f32(0.8)]
    assert O.l2_norm_rows([0.0, 0.0], 2, 0.1).tolist() == [0.0, 0.0]
    x = np.array([1.0, 2.0, 3.0], np.float32)
    scale = f32(1.0) / max(np.sqrt(f32(14.0)), f32(1e-6))
    assert bits(O.l2_norm_rows(x, 3, 1e-6)).tolist() == bits(x * scale).tolist()
    assert O.l2_norm_rows([3.0, 4.0, 6.0, 8.0], 2, 1e-6).tolist() == [f32(0.6), f32(0.8), f32(0.6), f32(0.8)]
    with pytest.raises(ValueError):
        O.l2_norm_rows([1.0, 2.0, 3.0], 2, 1e-6)


def _pairwise(vals):  # kernels.rs:27-42, written out
    level = list(vals)
    while len(level) > 1:
        nxt = [level[i] + level[i + 1] for i in range(0, len(level) - 1, 2)]
        if len(level) % 2:
            nxt.append(level[-1])
        level = nxt
    return level[0] if level else 0.0


def test_softmax_max_subtraction_and_partition():  # kernels.rs:562-593
    o1 = O.softmax([1000.0, 1001.0, 1002.0], 1.0)
    o2 = O.softmax([-2.0, -1.0, 0.0], 1.0)
    assert bits(o1).tolist() == bits(o2).tolist()
    e = [float(expf(v)) for v in (-2.0, -1.0, 0.0)]
    s = (e[0] + e[1]) + e[2]
    assert bits(o1).tolist() == bits([f32(v / s) for v in e]).tolist()
    assert abs((float(o1[0]) + float(o1[1])) + float(o1[2]) - 1.0) < 1e-7
    assert bits(O.softmax([-2.0, -1.0, 0.0], 2.0)).tolist() == bits(O.softmax([-4.0, -2.0, 0.0], 1.0)).tolist()


def test_softmax_denominator_is_the_pairwise_tree():
    rng = np.random.default_rng(2)
    for n in (1, 2, 5, 33, 1000):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        m = np.max(x)
        ef = np.array([math.exp(float(f32(v - m) * f32(0.7))) for v in x], np.float64).astype(np.float32)
        ref = [f32(float(v) / _pairwise([float(u) for u in ef])) for v in ef]
        got = O.softmax(x, 0.7)
        # exp: C expf vs exp in f64 rounded once may differ by an ulp; the
        # partition must not add more than that
        assert np.max(np.abs(bits(got).astype(np.int64) - bits(ref).astype(np.int64))) <= 2


def test_sigmoid_silu_softplus_f64_formulas():  # kernels.rs:626-661
    assert (O.sigmoid([0.0] * 3) == 0.5).all()
    assert (O.silu([0.0] * 3) == 0.0).all()
    assert O.softplus([0.0])[0] == f32(math.log(2.0))
    sig = 1.0 / (1.0 + math.exp(-1.0))
    assert bits(O.sigmoid([1.0])).tolist() == bits([sig]).tolist()
    assert bits(O.silu([1.0])).tolist() == bits([1.0 * sig]).tolist()
    sp = O.softplus([1.0])
    assert bits(sp).tolist() == bits([math.log(1.0 + math.e)]).tolist() and abs(sp[0] - 1.3132617) < 1e-6
    s = O.sigmoid([-1.0, 1.0])
    assert bits(s).tolist() == bits([1.0 / (1.0 + math.exp(1.0)), 1.0 / (1.0 + math.exp(-1.0))]).tolist()
    assert O.softplus([25.0])[0] == 25.0  # above 20: the identity branch


def test_ssm_conv_hand_values_and_f32_order():  # kernels.rs:695-730
    assert O.ssm_conv([1, 10, 2, 20, 3, 30], [1, 2, 3, 4], 2, 2).tolist() == [7.0, 100.0, 11.0, 160.0]
    assert O.ssm_conv([1e16, 1.0, -1e16, 1.0], [1.0] * 4, 4, 1).tolist() == [1.0]
    k = np.array([0.1, 0.2, 0.3, 0.4], np.float32)
    x = np.array([1.5, 2.5, 3.5, 4.5, 5.5, 6.5], np.float32)
    exp = []
    for t in range(2):
        for c in range(2):
            s = f32(0.0)
            for tau in range(2):
                s = f32(s + f32(x[(t + tau) * 2 + c] * k[tau * 2 + c]))
            exp.append(s)
    assert bits(O.ssm_conv(x, k, 2, 2)).tolist() == bits(exp).tolist()


def test_gdn_fused_step_hand_values():  # kernels.rs:800-857
    st, out = O.gdn_fused_step([1.0, 0.0, 0.0, 1.0], [1.0, 0.0], [1.0, 1.0], [3.0, 4.0], 0.0, 1.0, 1.0)
    assert st.tolist() == [3.0, 3.0, 2.0, 4.0] and out.tolist() == [3.0, 3.0]
    g = float(np.log(f32(0.5)))
    st2, out2 = O.gdn_fused_step(st, [1.0, 0.0], [1.0, 1.0], [3.0, 4.0], g, 1.0, 1.0)
    rep = st * expf(g)
    d0 = f32(3.0) - (rep[0] + rep[2])
    d1 = f32(4.0) - (rep[1] + rep[3])
    rep = rep + np.array([d0, d1, d0, d1], np.float32)
    assert abs(st2[0] - rep[0]) < 1e-6 and abs(out2[0] - rep[0]) < 1e-6 and abs(out2[1] - rep[1]) < 1e-6


def test_gdn_fused_step_scale_is_on_output_not_q():  # kernels.rs:859-881
    st, out = O.gdn_fused_step([3.0, 3.0, 2.0, 4.0], [1.0, 1.0], [1.0, 1.0], [3.0, 4.0], 0.0, 1.0, 2.0)
    assert st.tolist() == [1.0, 0.0, 0.0, 1.0] and out.tolist() == [2.0, 2.0]


def _gdn_py(state, q, k, v, gate, beta, scale):
    dim = len(q)
    S = np.array(state, np.float32).reshape(dim, dim).copy()
    S = (S * expf(gate)).astype(np.float32)
    d = np.zeros(dim, np.float32)
    for j in range(dim):
        s = 0.0
        for i in range(dim):
            s += float(f32(S[i, j] * k[i]))
        d[j] = f32(f32(v[j] - f32(s)) * f32(beta))
    for j in range(dim):
        for i in range(dim):
            S[i, j] = f32(S[i, j] + f32(k[i] * d[j]))
    out = np.zeros(dim, np.float32)
    for j in range(dim):
        s = 0.0
        for i in range(dim):
            s += float(f32(S[i, j] * q[i]))
        out[j] = f32(f32(s) * f32(scale))
    return S.reshape(-1), out


def test_gdn_fused_step_replicates_documented_f32_chain():  # kernels.rs:883-921, and a random 16-dim head
    q = np.array([0.25, -0.5, 0.75], np.float32)
    k = np.array([-0.125, 0.5, 0.375], np.float32)
    v = np.array([1.0, -2.0, 0.5], np.float32)
    st0 = np.eye(3, dtype=np.float32).reshape(-1)
    st, out = O.gdn_fused_step(st0, q, k, v, 0.0, 0.8, 0.0625)
    rs, ro = _gdn_py(st0, q, k, v, 0.0, 0.8, 0.0625)
    assert bits(st).tolist() == bits(rs).tolist() and bits(out).tolist() == bits(ro).tolist()
    rng = np.random.default_rng(3)
    dim = 16
    st0 = rng.standard_normal(dim * dim).astype(np.float32)
    q, k, v = (rng.standard_normal(dim).astype(np.float32) for _ in range(3))
    st, out = O.gdn_fused_step(st0, q, k, v, -0.3, 0.7, 0.25)
    rs, ro = _gdn_py(st0, q, k, v, -0.3, 0.7, 0.25)
    assert bits(st).tolist() == bits(rs).tolist() and bits(out).tolist() == bits(ro).tolist()


def _rot(x0, x1, a):
    s, c = math.sin(a), math.cos(a)
    fma = _libm.fma  # Rust's f64::mul_add: one rounding
    return f32(fma(c, float(x0), -(s * float(x1)))), f32(fma(s, float(x0), c * float(x1)))


def test_rope_llama_identity_cases():  # kernels.rs:513-539
    x = [1.5, -2.25, 3.0, 4.0]
    assert O.rope_llama(x, [0.5, 0.25], 0).tolist() == x
    assert O.rope_llama(x, [0.0, 0.0], 7).tolist() == x
    half_pi = f32(math.pi / 2)
    got = O.rope_llama([1.0, 0.0], [half_pi], 1)
    e0, e1 = _rot(1.0, 0.0, float(half_pi))
    assert bits(got).tolist() == bits([e0, e1]).tolist() and got[1] == 1.0


def test_rope_neox_identity_and_rotation():  # kernels.rs:541-560
    x = [1.5, -2.25, 3.0, 4.0]
    assert O.rope_neox(x, [0.5, 0.25], 0).tolist() == x
    half_pi = f32(math.pi / 2)
    got = O.rope_neox([1.0, 99.0, 0.0, 99.0], [half_pi, 0.0], 1)
    e0, e2 = _rot(1.0, 0.0, float(half_pi))
    assert bits(got[[0, 2]]).tolist() == bits([e0, e2]).tolist() and got[1] == 99.0 and got[3] == 99.0


def test_rope_imrope_interleaved_pairs():  # kernels.rs:732-779
    got = O.rope_imrope([1.0, 99.0, 0.0, 99.0, 7.0, 8.0], 4, 0.01, 1)
    e0, e2 = _rot(1.0, 0.0, 1.0)
    assert bits(got[[0, 2]]).tolist() == bits([e0, e2]).tolist()
    assert got[[1, 3, 4, 5]].tolist() == [99.0, 99.0, 7.0, 8.0]
    x = [1.5, -2.25, 3.0, 4.0]
    assert O.rope_imrope(x, 4, 0.01, 0).tolist() == x
    orig = np.arange(12, dtype=np.float32)
    got = O.rope_imrope(orig, 12, 0.01, 1)
    r0, r6 = _rot(orig[0], orig[6], 1.0)
    r3, r9 = _rot(orig[3], orig[9], 0.01 ** 3)
    exp = orig.copy()
    exp[[0, 6, 3, 9]] = [r0, r6, r3, r9]
    assert bits(got).tolist() == bits(exp).tolist()


def test_rope_imrope_angle_is_the_running_product():
    """Pair ic's angle is pos * theta multiplied ic times, one rounding each."""
    n_rot, theta, pos = 64, 0.8659643, 37
    x = np.random.default_rng(4).standard_normal(80).astype(np.float32)
    got = O.rope_imrope(x, n_rot, theta, pos)
    exp = x.copy()
    angle = float(pos)
    for ic in range(n_rot // 2):
        if ic % 3 == 0:
            exp[ic], exp[ic + n_rot // 2] = _rot(x[ic], x[ic + n_rot // 2], angle)
        angle *= theta
    assert bits(got).tolist() == bits(exp).tolist()


def _attn_f64(q, kc, vc, n_ctx, nh, nhkv, hd, scale):
    """A float64 restatement for closeness (not bit-level) checks."""
    G = nh // nhkv
    K = kc[: n_ctx * nhkv * hd].reshape(n_ctx, nhkv, hd).astype(np.float64)
    V = vc[: n_ctx * nhkv * hd].reshape(n_ctx, nhkv, hd).astype(np.float64)
    out = np.zeros((nh, hd))
    for h in range(nh):
        s = K[:, h // G, :] @ q[h * hd:(h + 1) * hd].astype(np.float64) * scale
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ V[:, h // G, :]
    return out.reshape(-1)


def test_attn_decode_single_position_returns_v_of_the_heads_kv():  # qwen35_forward.rs:639-671
    """n_ctx = 1: soft = [1.0] and out_h = V[kv(h)] exactly; kv(h) = h / group
    (consecutive heads share a kv head, not h % n_head_kv)."""
    rng = np.random.default_rng(20)
    nh, nhkv, hd = 4, 2, 8
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kc = rng.standard_normal(nhkv * hd).astype(np.float32)
    vc = rng.standard_normal(nhkv * hd).astype(np.float32)
    out, soft = O.attn_decode(q, kc, vc, 1, nh, nhkv, hd, 0.125)
    assert soft.tolist() == [1.0] * nh
    V = vc.reshape(nhkv, hd)
    assert bits(out).tolist() == bits(np.concatenate([V[0], V[0], V[1], V[1]])).tolist()


def test_attn_decode_value_sum_is_sequential_in_position():
    """Equal keys give soft = 1/4 exactly; the column [2^62, 1, -2^62, 1]
    then sums to 0.25 in the reference's sequential order (the pairwise
    order, or the reversed one, gives 0)."""
    hd, n_ctx = 4, 4
    q = np.ones(hd, np.float32)
    kc = np.ones(n_ctx * hd, np.float32)
    col = [2.0 ** 62, 1.0, -(2.0 ** 62), 1.0]
    vc = np.array([[c] * hd for c in col], np.float32).reshape(-1)
    out, soft = O.attn_decode(q, kc, vc, n_ctx, 1, 1, hd, 1.0)
    assert soft.tolist() == [0.25] * 4
    assert out.tolist() == [0.25] * hd


def test_attn_decode_scores_use_the_pairwise_dot():
    """Key 0's products [2^60, 1, -2^60, 1] sum to 0 in the pairwise tree
    (1 sequentially); key 1 scores 0: the weights are [0.5, 0.5] only if the
    score is dot_f32's pairwise sum."""
    hd = 4
    q = np.ones(hd, np.float32)
    kc = np.array([2.0 ** 60, 1.0, -(2.0 ** 60), 1.0, 0, 0, 0, 0], np.float32)
    vc = np.array([1.0] * hd + [0.0] * hd, np.float32)
    out, soft = O.attn_decode(q, kc, vc, 2, 1, 1, hd, 1.0)
    assert soft.tolist() == [0.5, 0.5]
    assert out.tolist() == [0.5] * hd


def test_attn_decode_close_to_float64_attention():
    rng = np.random.default_rng(21)
    for n_ctx, nh, nhkv, hd in [(1, 2, 1, 16), (7, 4, 2, 32), (50, 8, 2, 64)]:
        q = rng.standard_normal(nh * hd).astype(np.float32)
        kc = rng.standard_normal(n_ctx * nhkv * hd).astype(np.float32)
        vc = rng.standard_normal(n_ctx * nhkv * hd).astype(np.float32)
        scale = 1.0 / math.sqrt(hd)
        out, soft = O.attn_decode(q, kc, vc, n_ctx, nh, nhkv, hd, scale)
        np.testing.assert_allclose(out, _attn_f64(q, kc, vc, n_ctx, nh, nhkv, hd, scale), rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(soft.reshape(nh, n_ctx).sum(axis=1), 1.0, rtol=1e-6)


def test_matmul_exact_acc_semantics_and_order_adversary():  # kernels.rs:488-511
    a = [1.0, 2.0, 3.0, 4.0, 5.0, 6.0]
    b = [7.0, 8.0, 9.0, 10.0, 11.0, 12.0]
    acc = O.matmul_f32_acc(np.zeros(4), a, b, 2, 3, 2)
    assert acc.tolist() == [58.0, 64.0, 139.0, 154.0]
    assert O.matmul_f32_acc(acc, a, b, 2, 3, 2).tolist() == [116.0, 128.0, 278.0, 308.0]
    assert O.matmul_f32_acc([0.0], [1e19, 1.0, -1e19, 1.0], [1.0] * 4, 1, 4, 1).tolist() == [0.0]


def test_matmul_is_pairwise_then_one_rounding():
    rng = np.random.default_rng(22)
    m, k, n = 3, 37, 2
    a = (rng.standard_normal(m * k) * 2.0 ** rng.integers(-20, 20, m * k)).astype(np.float32)
    b = rng.standard_normal(k * n).astype(np.float32)
    acc0 = rng.standard_normal(m * n).astype(np.float32)
    got = O.matmul_f32_acc(acc0, a, b, m, k, n)
    A, B = a.reshape(m, k).astype(np.float64), b.reshape(k, n).astype(np.float64)
    for i in range(m):
        for j in range(n):
            s = _pairwise([A[i, l] * B[l, j] for l in range(k)])
            assert bits([got[i * n + j]]).tolist() == bits([np.float32(float(acc0[i * n + j]) + s)]).tolist()


def test_gelu_tanh_hand_values():  # kernels.rs:612-623
    out = O.gelu_tanh([0.0, 1.0])
    assert out[0] == 0.0
    S, Cc, t = 0.7978845608028654, 0.044715, 1.0
    e = f32(0.5 * t * (1.0 + math.tanh(S * (t + Cc * t * t * t))))
    assert bits(out[1:]).tolist() == bits([e]).tolist() and abs(out[1] - 0.84119199) < 1e-5
    x = np.linspace(-6, 6, 101).astype(np.float32)
    ref = [f32(0.5 * float(v) * (1.0 + math.tanh(S * (float(v) + Cc * float(v) * float(v) * float(v))))) for v in x]
    assert bits(O.gelu_tanh(x)).tolist() == bits(ref).tolist()


def test_embedding_lookup_copies_rows_and_refuses_out_of_range():  # kernels.rs:780-798
    table = np.array([i * 10.0 + (i % 3) for i in range(12)], np.float32)
    out = O.embedding_lookup(table, [0, 3, 1], 3)
    assert out.tolist() == table[0:3].tolist() + table[9:12].tolist() + table[3:6].tolist()
    with pytest.raises(ValueError, match="status 5"):
        O.embedding_lookup(np.zeros(6, np.float32), [0, 99], 2)
    with pytest.raises(ValueError, match="status 1"):
        O.embedding_lookup(np.zeros(7, np.float32), [0], 2)

