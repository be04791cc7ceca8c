"""GPU parity of the per-layer ops (include/uq_ops.h) against the oracle.

Bars (see uq_ops.h):
  * bit-exact: rmsnorm, l2_norm_rows (including inputs whose mean sits on an
    f32 rounding boundary, which take the sequential replay), ssm_conv,
    gdn_fused_step with exp(gate) exact, and the rope rotations;
  * within 2 ulp of the oracle's C library expf / logf: sigmoid, silu,
    softplus, softmax and gdn_fused_step with a general gate; nearly all
    elements bit-equal (the device's exp / log are correctly rounded, the C
    library's are not always).
"""
import numpy as np
import pytest

import oracle as O
import uq
from uq import ops

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)


def assert_bitwise(got, ref, what):
    g, r = bits(got), bits(ref)
    bad = np.nonzero(g != r)[0]
    assert bad.size == 0, f"{what}: {bad.size} differ, first {bad[:5].tolist()}"


def assert_ulp(got, ref, max_ulp, min_equal, what):
    g, r = bits(got), bits(ref)
    d = np.abs(g - r)
    assert d.max() <= max_ulp, f"{what}: max ulp {d.max()} at {int(np.argmax(d))}"
    frac = float(np.mean(d == 0))
    assert frac >= min_equal, f"{what}: only {frac:.4f} bit-equal"


def dev(a):
    return uq.DeviceArray.from_numpy(np.ascontiguousarray(a, np.float32))


@pytest.mark.parametrize("n", [1, 7, 300, 4096, 5000, 12288])
def test_rmsnorm_bit_exact(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 40.0], n)).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    assert_bitwise(ops.rmsnorm(x, w, 1e-6), O.rmsnorm(x, w, 1e-6), f"rmsnorm n={n}")


def test_rmsnorm_rows_on_device_and_the_boundary_replay():
    rng = np.random.default_rng(5)
    n, rows = 4096, 9
    X = rng.standard_normal((rows, n)).astype(np.float32)
    # row 8: mean = 2^-10 (1 + 2^-24) exactly, the midpoint between two f32 values,
    # so the tree-sum bound cannot decide and the sequential loop runs
    X[8] = 0.0
    X[8, 4092:] = [1.0, 1.0, 1.0, np.nextafter(np.float32(1.0), np.float32(2.0))]
    w = rng.standard_normal(n).astype(np.float32)
    dx, dw, dy = dev(X), dev(w), uq.DeviceArray(4 * n * rows)
    ops.rmsnorm_d(dy, dx, dw, n, rows, 1e-6)
    uq.synchronize()
    got = dy.download(np.float32, n * rows).reshape(rows, n)
    for r in range(rows):
        assert_bitwise(got[r], O.rmsnorm(X[r], w, 1e-6), f"rmsnorm row {r}")
    # the small case of the midpoint: [1, 1, 1, 1+2^-23] with eps 0
    x4 = np.array([1.0, 1.0, 1.0, np.nextafter(np.float32(1.0), np.float32(2.0))], np.float32)
    assert_bitwise(ops.rmsnorm(x4, np.ones(4, np.float32), 0.0), O.rmsnorm(x4, np.ones(4, np.float32), 0.0),
                   "rmsnorm midpoint")


def undecided_row(rng, n, above):
    """A row of n random values whose sequential f64 sum of f32 squares (the
    reference's order) lies a few ulps from n times an f32 midpoint, well
    inside the device's bound, so the tree-sum bound cannot decide the mean
    and the device replays the sequential loop; above: the sum lands on the
    side of the midpoint that rounds up (a replay that is skipped, or drops
    or repeats a term, gives the wrong bits). The last two values steer the
    sum."""
    x = rng.standard_normal(n).astype(np.float32)
    P = 0.0
    for v in x[:n - 2]:
        P += float(np.float32(v) * np.float32(v))
    a = np.float32(P / n * (1 + 2.0 ** -16))
    mid = (float(a) + float(np.nextafter(a, np.float32(np.inf)))) / 2  # exact in f64
    T = mid * n
    e = (n + 66) * 2.0 ** -52 * T
    target = T + (3 if above else -3) * 2.0 ** -52 * T
    v = np.float32(np.sqrt((target - P) * (1 - 2.0 ** -20)))
    P1 = P + float(v * v)
    w = np.float32(np.sqrt(target - P1))
    x[n - 2], x[n - 1] = v, w
    S = P1 + float(w * w)
    assert abs(S - T) < e / 4 and (S > T) == above, (S, T, e)
    return x


@pytest.mark.parametrize("n", [4096, 5000, 12288])
def test_rmsnorm_rows_replay_the_sequential_sum(n):
    """Rows whose mean the bound cannot decide, the sum over thousands of
    random squares: the replay's result must be the reference's bit for bit
    (both sides of the midpoint; decided rows between them)."""
    rng = np.random.default_rng(n + 17)
    X = np.stack([undecided_row(rng, n, above=r % 2 == 0) if r % 3 != 2 else rng.standard_normal(n).astype(np.float32)
                  for r in range(6)])
    w = rng.standard_normal(n).astype(np.float32)
    dx, dw, dy = dev(X), dev(w), uq.DeviceArray(4 * n * len(X))
    ops.rmsnorm_d(dy, dx, dw, n, len(X), 1e-30)
    uq.synchronize()
    got = dy.download(np.float32, n * len(X)).reshape(len(X), n)
    for r in range(len(X)):
        assert_bitwise(got[r], O.rmsnorm(X[r], w, 1e-30), f"rmsnorm replay row {r} n={n}")
    for a in (dx, dw, dy):
        a.free()


def test_l2_norm_rows_bit_exact_and_boundary():
    rng = np.random.default_rng(6)
    dim, rows = 128, 64
    X = (rng.standard_normal(rows * dim) * 3).astype(np.float32)
    X[:dim] = 0.0
    X[dim - 4:dim] = [1.0, 1.0, 1.0, np.nextafter(np.float32(1.0), np.float32(2.0))]  # sum = 4 + 2^-22: f32 midpoint
    assert_bitwise(ops.l2_norm_rows(X, dim, 1e-6), O.l2_norm_rows(X, dim, 1e-6), "l2_norm_rows host")
    d = dev(X)
    ops.l2_norm_rows_d(d, len(X), dim, 1e-6)
    uq.synchronize()
    assert_bitwise(d.download(np.float32, len(X)), O.l2_norm_rows(X, dim, 1e-6), "l2_norm_rows device")


@pytest.mark.parametrize("n", [1, 3, 1000, 8192])
def test_softmax_within_2_ulp(n):
    rng = np.random.default_rng(n + 1)
    x = (rng.standard_normal(n) * 5).astype(np.float32)
    assert_ulp(ops.softmax(x, 0.125), O.softmax(x, 0.125), 2, 0.99, f"softmax n={n}")


def test_softmax_reference_case_and_device_rows():
    assert_bitwise(ops.softmax([1000.0, 1001.0, 1002.0], 1.0), O.softmax([1000.0, 1001.0, 1002.0], 1.0), "kat")
    rng = np.random.default_rng(8)
    n, rows = 777, 16
    X = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    dx, dy = dev(X), uq.DeviceArray(4 * n * rows)
    ops.softmax_d(dy, dx, n, rows, 0.5)
    uq.synchronize()
    got = dy.download(np.float32, n * rows).reshape(rows, n)
    for r in range(rows):
        assert_ulp(got[r], O.softmax(X[r], 0.5), 2, 0.99, f"softmax row {r}")


def softmax_model(x, scale):
    """The device's method for softmax: f32 steps, each exp the f64 function
    rounded once to f32, the denominator the reference's pairwise tree
    (kernels.rs:21-42: pairs (2i, 2i+1), an odd tail carried up) in f64."""
    f = np.float32
    x = np.asarray(x, f)
    e = np.exp(((x - x.max()) * f(scale)).astype(np.float64)).astype(f)
    lv = [float(v) for v in e]
    while len(lv) > 1:
        lv = [lv[i] + lv[i + 1] if i + 1 < len(lv) else lv[i] for i in range(0, len(lv), 2)]
    return (e.astype(np.float64) / lv[0]).astype(f)


@pytest.mark.parametrize("n", [1, 15, 16, 17, 100, 777, 1024, 1025, 3000])
def test_softmax_rows_equal_the_pairwise_model(n):
    """Rows of up to 1024 take one wave each (16-element lane trees, then
    the wave's tree), longer rows the workgroup's LDS tree: both give the
    reference's pairwise denominator, bit for bit against the model."""
    rng = np.random.default_rng(n + 3)
    rows = 5
    X = (rng.standard_normal((rows, n)) * 4).astype(np.float32)
    dx, dy = dev(X), uq.DeviceArray(4 * n * rows)
    ops.softmax_d(dy, dx, n, rows, 0.25)
    uq.synchronize()
    got = dy.download(np.float32, n * rows).reshape(rows, n)
    for r in range(rows):
        assert_bitwise(got[r], softmax_model(X[r], 0.25), f"softmax n={n} row {r}")
    for a_ in (dx, dy):
        a_.free()


def unary_cr(name, x):
    """The device's method: each f32 exp / log is the f64 function rounded
    once to f32; the other steps are single f32 operations."""
    f = np.float32
    x = np.asarray(x, np.float32)
    if name == "softplus":
        e = np.exp(x.astype(np.float64)).astype(f)
        return np.where(x > f(20), x, np.log((f(1) + e).astype(np.float64)).astype(f))
    e = np.exp(-x.astype(np.float64)).astype(f)
    return (f(1) if name == "sigmoid" else x) / (f(1) + e)


@pytest.mark.parametrize("n", [8193, 16384, 16385, 40000])
def test_softmax_rows_beyond_one_chunk(n):
    """Rows longer than the 8192-value LDS chunk: the denominator is the tree
    over chunk sums, which must equal the pairwise tree over the whole row."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 4).astype(np.float32)
    assert_ulp(ops.softmax(x, 0.3), O.softmax(x, 0.3), 2, 0.99, f"softmax n={n}")
    # in place on the device, two rows
    X = np.stack([x, x[::-1]]).astype(np.float32)
    d = dev(X)
    ops.softmax_d(d, d, n, 2, 0.3)
    uq.synchronize()
    got = d.download(np.float32, 2 * n).reshape(2, n)
    assert_ulp(got[0], O.softmax(X[0], 0.3), 2, 0.99, "softmax in place row 0")
    assert_ulp(got[1], O.softmax(X[1], 0.3), 2, 0.99, "softmax in place row 1")


@pytest.mark.parametrize("name", ["sigmoid", "silu", "softplus"])
def test_unary_within_2_ulp(name):
    """Within 2 ulp of the oracle (the C library's expf / logf, as the
    reference calls them); glibc's logf is not correctly rounded for about
    0.75% of the arguments of softplus here, so bit-equality with the oracle
    is only required of 99%. Against the correctly rounded f64 model of the
    device's own method the bar is bit-equality but for rare near-midpoint
    arguments."""
    rng = np.random.default_rng(9)
    x = np.concatenate([rng.uniform(-30, 30, 200000), [0.0, -0.0, 1.0, -1.0, 20.0, 20.5, -88.0, 88.0]]).astype(np.float32)
    ref, cr = getattr(O, name)(x), unary_cr(name, x)
    got = getattr(ops, name)(x)
    assert_ulp(got, ref, 2, 0.99, f"{name} host")
    assert_ulp(got, cr, 1, 0.9999, f"{name} host vs f64 model")
    d, y = dev(x), uq.DeviceArray(4 * len(x))
    ops.unary_d(name, y, d, len(x))
    uq.synchronize()
    got = y.download(np.float32, len(x))
    assert_ulp(got, ref, 2, 0.99, f"{name} device")
    assert_ulp(got, cr, 1, 0.9999, f"{name} device vs f64 model")


@pytest.mark.parametrize("d_conv,channels,n_t", [(4, 8192, 1), (4, 8192, 7), (2, 2, 2)])
def test_ssm_conv_bit_exact(d_conv, channels, n_t):
    rng = np.random.default_rng(channels + n_t)
    x = rng.standard_normal((d_conv - 1 + n_t) * channels).astype(np.float32)
    k = rng.standard_normal(d_conv * channels).astype(np.float32)
    ref = O.ssm_conv(x, k, d_conv, channels)
    assert_bitwise(ops.ssm_conv(x, k, d_conv, channels), ref, "ssm_conv host")
    dx, dk, dy = dev(x), dev(k), uq.DeviceArray(4 * len(ref))
    ops.ssm_conv_d(dy, dx, len(x), dk, d_conv, channels)
    uq.synchronize()
    assert_bitwise(dy.download(np.float32, len(ref)), ref, "ssm_conv device")


@pytest.mark.parametrize("dim", [128, 64, 100, 200])
def test_gdn_fused_step_heads(dim):
    """dim <= 128: the column-in-registers kernel (one or two elements of
    q and k per lane, a partial last wave at 100); 200: the general one."""
    rng = np.random.default_rng(10 + dim)
    heads = 8
    S = (rng.standard_normal((heads, dim, dim)) * 0.1).astype(np.float32)
    q, k, v = (rng.standard_normal((heads, dim)).astype(np.float32) for _ in range(3))
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    gate = np.zeros(heads, np.float32)  # exp(0) = 1 on both sides: bit-exact
    gate[4:] = rng.uniform(-2, 0, 4)    # general gates: exp may differ by an ulp
    beta = rng.uniform(0, 1, heads).astype(np.float32)
    ds, dq, dk, dv, dg, db = dev(S), dev(q), dev(k), dev(v), dev(gate), dev(beta)
    dout = uq.DeviceArray(4 * heads * dim)
    ops.gdn_fused_step_d(ds, dout, dq, dk, dv, dg, db, dim, heads, 0.0884)
    uq.synchronize()
    gs = ds.download(np.float32, heads * dim * dim).reshape(heads, dim * dim)
    go = dout.download(np.float32, heads * dim).reshape(heads, dim)
    for h in range(heads):
        rs, ro = O.gdn_fused_step(S[h].reshape(-1), q[h], k[h], v[h], float(gate[h]), float(beta[h]), 0.0884)
        if h < 4:
            assert_bitwise(gs[h], rs, f"gdn state head {h}")
            assert_bitwise(go[h], ro, f"gdn out head {h}")
        else:
            np.testing.assert_allclose(gs[h], rs, rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(go[h], ro, rtol=1e-4, atol=1e-5)
    # one head through the host mirror
    rs, ro = O.gdn_fused_step(S[0].reshape(-1), q[0], k[0], v[0], 0.0, float(beta[0]), 0.5)
    hs, ho = ops.gdn_fused_step(S[0].reshape(-1), q[0], k[0], v[0], 0.0, float(beta[0]), 0.5)
    assert_bitwise(hs, rs, "gdn host state")
    assert_bitwise(ho, ro, "gdn host out")


def test_gdn_fused_step_midpoint_dots_take_the_ordered_sum():
    """Columns whose k- and q-dots are exact f32 midpoints (1 + 2^-24): the
    parallel partial sums cannot decide the rounding, so the kernel sums in
    the reference's order; the results stay bit-exact."""
    dim, heads = 128, 2
    S = np.zeros((heads, dim, dim), np.float32)
    S[:, 0, :] = 1.0
    S[:, 1, :] = 2.0 ** -24
    q = np.zeros((heads, dim), np.float32)
    k = np.zeros((heads, dim), np.float32)
    q[:, :2] = 1.0
    k[:, :2] = 1.0
    v = np.full((heads, dim), 3.0, np.float32)
    gate, beta = np.zeros(heads, np.float32), np.array([0.5, 0.25], np.float32)
    ds, dq, dk, dv, dg, db = dev(S), dev(q), dev(k), dev(v), dev(gate), dev(beta)
    dout = uq.DeviceArray(4 * heads * dim)
    ops.gdn_fused_step_d(ds, dout, dq, dk, dv, dg, db, dim, heads, 1.0)
    uq.synchronize()
    gs = ds.download(np.float32, heads * dim * dim).reshape(heads, dim * dim)
    go = dout.download(np.float32, heads * dim).reshape(heads, dim)
    for h in range(heads):
        rs, ro = O.gdn_fused_step(S[h].reshape(-1), q[h], k[h], v[h], 0.0, float(beta[h]), 1.0)
        assert_bitwise(gs[h], rs, f"midpoint state head {h}")
        assert_bitwise(go[h], ro, f"midpoint out head {h}")


@pytest.mark.parametrize("kind", ["llama", "neox"])
def test_rope_freq(kind):
    rng = np.random.default_rng(11)
    n, rows, pos = 256, 32, 1234
    freqs = (10000.0 ** (-np.arange(n // 2) * 2.0 / n)).astype(np.float32)
    X = rng.standard_normal((rows, n)).astype(np.float32)
    ref = np.stack([getattr(O, f"rope_{kind}")(X[r], freqs, pos) for r in range(rows)])
    assert_ulp(getattr(ops, f"rope_{kind}")(X[0], freqs, pos), ref[0], 1, 0.999, f"rope {kind} host")
    d, df = dev(X), dev(freqs)
    ops.rope_d(kind, d, n, rows, df, pos)
    uq.synchronize()
    assert_ulp(d.download(np.float32, n * rows), ref.reshape(-1), 1, 0.999, f"rope {kind} device")


def test_rope_imrope():
    rng = np.random.default_rng(12)
    n, n_rot, rows, pos = 256, 64, 24, 4321
    theta = float(np.float32(10000.0) ** np.float32(-2.0 / n_rot))
    X = rng.standard_normal((rows, n)).astype(np.float32)
    ref = np.stack([O.rope_imrope(X[r], n_rot, theta, pos) for r in range(rows)])
    assert_ulp(ops.rope_imrope(X[0], n_rot, theta, pos), ref[0], 1, 0.999, "imrope host")
    d = dev(X)
    ops.rope_imrope_d(d, n, rows, n_rot, theta, pos)
    uq.synchronize()
    assert_ulp(d.download(np.float32, n * rows), ref.reshape(-1), 1, 0.999, "imrope device")
    kat = ops.rope_imrope([1.0, 99.0, 0.0, 99.0, 7.0, 8.0], 4, 0.01, 1)
    assert_bitwise(kat, O.rope_imrope([1.0, 99.0, 0.0, 99.0, 7.0, 8.0], 4, 0.01, 1), "imrope kat")


def attn_case(seed, n_ctx, nh, nhkv, hd, spare=0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kc = rng.standard_normal((n_ctx + spare) * nhkv * hd).astype(np.float32)
    vc = rng.standard_normal((n_ctx + spare) * nhkv * hd).astype(np.float32)
    return q, kc, vc


def check_attn(q, kc, vc, n_ctx, nh, nhkv, hd, scale, what, bit_exact_soft=False):
    ref, rsoft = O.attn_decode(q, kc, vc, n_ctx, nh, nhkv, hd, scale)
    dq, dk, dv = dev(q), dev(kc), dev(vc)
    dout, dsoft = uq.DeviceArray(4 * nh * hd), uq.DeviceArray(4 * nh * n_ctx)
    ops.attn_decode_d(dout, dsoft, dq, dk, dv, n_ctx, nh, nhkv, hd, scale)
    uq.synchronize()
    got, soft = dout.download(np.float32, nh * hd), dsoft.download(np.float32, nh * n_ctx)
    if bit_exact_soft:
        assert_bitwise(soft, rsoft, f"{what} soft")
        assert_bitwise(got, ref, f"{what} out")
    else:
        # softmax's expf may differ from the C library's by an ulp; where the
        # weights agree bit for bit, out must too
        assert_ulp(soft, rsoft, 2, 0.99, f"{what} soft")
        for h in range(nh):
            if np.array_equal(bits(soft[h * n_ctx:(h + 1) * n_ctx]), bits(rsoft[h * n_ctx:(h + 1) * n_ctx])):
                assert_bitwise(got[h * hd:(h + 1) * hd], ref[h * hd:(h + 1) * hd], f"{what} head {h}")
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
    return got


@pytest.mark.parametrize("n_ctx,nh,nhkv,hd", [(1, 16, 4, 256), (7, 16, 4, 256), (300, 16, 4, 256),
                                              (2049, 16, 4, 256), (33, 8, 8, 64), (100, 16, 2, 128),
                                              (65, 8, 1, 512), (50, 6, 2, 64), (40, 4, 2, 128), (70, 10, 2, 64)])
def test_attn_decode_matches_the_reference_loop(n_ctx, nh, nhkv, hd):
    q, kc, vc = attn_case(n_ctx * 7 + hd, n_ctx, nh, nhkv, hd, spare=3)  # caches longer than n_ctx, as in a session
    check_attn(q, kc, vc, n_ctx, nh, nhkv, hd, 1.0 / np.sqrt(hd), f"attn n_ctx={n_ctx} hd={hd}")
    if n_ctx == 300:
        out = ops.attn_decode(q, kc, vc, n_ctx, nh, nhkv, hd, 1.0 / np.sqrt(hd))
        ref, _ = O.attn_decode(q, kc, vc, n_ctx, nh, nhkv, hd, 1.0 / np.sqrt(hd))
        np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_attn_decode_order_adversaries_take_the_replay():
    """Equal keys (weights exactly 1/n_ctx, so bit-exact) and value columns
    with cancellation: [2^62, 1, -2^62, 1] sums to 0.25 only in sequential
    order, so the parallel bound cannot decide and the lane replays; the
    pairwise score adversary of dot_f32 gives weights [0.5, 0.5]."""
    hd, n_ctx = 64, 4
    q = np.ones(hd, np.float32)
    kc = np.ones(n_ctx * hd, np.float32)
    col = np.array([2.0 ** 62, 1.0, -(2.0 ** 62), 1.0], np.float32)
    vc = np.repeat(col, hd).astype(np.float32)
    vc[1::2] *= -1.0  # half the columns sum to -0.25 ... mixed signs across lanes
    got = check_attn(q, kc, vc, n_ctx, 1, 1, hd, 1.0, "adversary", bit_exact_soft=True)
    assert set(np.abs(got).tolist()) == {0.25}
    kq = np.zeros(2 * hd, np.float32)
    kq[:4] = [2.0 ** 60, 1.0, -(2.0 ** 60), 1.0]
    vv = np.concatenate([np.ones(hd), np.zeros(hd)]).astype(np.float32)
    got = check_attn(q, kq, vv, 2, 1, 1, hd, 1.0, "score adversary", bit_exact_soft=True)
    assert got.tolist() == [0.5] * hd


@pytest.mark.parametrize("cols", [(0,), (5, 9, 63), (1, 2, 3, 4, 5, 6, 7)])
def test_attn_decode_replays_a_few_columns_over_a_long_context(cols):
    """Equal weights over 300 positions; the listed value columns hold
    [2^62, 1, -2^62, 1, 0, ...], whose sum is the weight only in sequential
    order, the others N(0,1). Up to four such columns per wave are replayed
    by the whole wave one at a time, more by their own lanes: both must give
    the reference's sequential sum."""
    hd, n_ctx = 64, 300
    rng = np.random.default_rng(len(cols))
    q = np.ones(hd, np.float32)
    kc = np.ones(n_ctx * hd, np.float32)
    vc = rng.standard_normal((n_ctx, hd)).astype(np.float32)
    for c in cols:
        vc[:, c] = 0.0
        vc[:4, c] = [2.0 ** 62, 1.0, -(2.0 ** 62), 1.0]
    got = check_attn(q, kc, vc.reshape(-1), n_ctx, 1, 1, hd, 1.0, f"replay {cols}", bit_exact_soft=True)
    w = np.float32(got[cols[0]])
    assert all(got[c] == w for c in cols) and w > 0


def test_gelu_tanh_within_1_ulp():
    rng = np.random.default_rng(23)
    x = np.concatenate([rng.uniform(-8, 8, 100000), [0.0, -0.0, 1.0, -1.0, 30.0, -30.0]]).astype(np.float32)
    ref = O.gelu_tanh(x)
    assert_ulp(ops.gelu_tanh(x), ref, 1, 0.999, "gelu_tanh host")
    d, y = dev(x), uq.DeviceArray(4 * len(x))
    ops.unary_d("gelu_tanh", y, d, len(x))
    uq.synchronize()
    assert_ulp(y.download(np.float32, len(x)), ref, 1, 0.999, "gelu_tanh device")
    assert ops.gelu_tanh([0.0, 1.0])[0] == 0.0


@pytest.mark.parametrize("m,k,n", [(2, 3, 2), (1, 4, 1), (5, 1000, 7), (3, 4097, 2), (2, 4096 * 3 + 65, 3),
                                   (1, 64 ** 3, 1), (4, 0, 3)])
def test_matmul_f32_acc_bit_exact(m, k, n):
    """Wide exponents make the f64 sums order-sensitive: any order but the
    pairwise tree (including across the 64- and 4096-chunks) shows in f32."""
    rng = np.random.default_rng(m * 1000 + k + n)
    if (m, k, n) == (2, 3, 2):
        a, b = np.arange(1, 7, dtype=np.float32), np.arange(7, 13, dtype=np.float32)
    elif (m, k, n) == (1, 4, 1):
        a, b = np.array([1e19, 1.0, -1e19, 1.0], np.float32), np.ones(4, np.float32)
    else:
        a = (rng.standard_normal(m * k) * 2.0 ** rng.integers(-24, 24, m * k)).astype(np.float32)
        b = rng.standard_normal(k * n).astype(np.float32)
    acc = rng.standard_normal(m * n).astype(np.float32) if k > 4 else np.zeros(m * n, np.float32)
    ref = O.matmul_f32_acc(acc, a, b, m, k, n)
    assert_bitwise(ops.matmul_f32_acc(acc, a, b, m, k, n), ref, f"matmul host {m}x{k}x{n}")
    dacc, da, db = dev(acc), dev(a if k else np.zeros(1)), dev(b if k else np.zeros(1))
    ops.matmul_f32_acc_d(dacc, da, db, m, k, n)
    uq.synchronize()
    assert_bitwise(dacc.download(np.float32, m * n), ref, f"matmul device {m}x{k}x{n}")


def test_embedding_lookup_rows_bit_exact():
    rng = np.random.default_rng(24)
    vocab, dim = 1000, 384
    table = rng.standard_normal(vocab * dim).astype(np.float32)
    ids = rng.integers(0, vocab, 300).astype(np.uint32)  # crosses the 256-id launch chunk
    ref = O.embedding_lookup(table, ids, dim)
    assert_bitwise(ops.embedding_lookup(table, ids, dim), ref, "embedding_lookup host")
    dt, dy = dev(table), uq.DeviceArray(4 * len(ref))
    ops.embedding_lookup_d(dy, dt, len(table), ids, dim)
    uq.synchronize()
    assert_bitwise(dy.download(np.float32, len(ref)), ref, "embedding_lookup device")
    with pytest.raises(uq.UqError) as e:
        ops.embedding_lookup(table, [0, vocab], dim)
    assert e.value.kind == "TOKEN"

