"""Shared helpers for the parity tests."""
import numpy as np

ATOL, RTOL = 1e-4, 1e-3  # |y - r| <= ATOL + RTOL * |r| (gemv_quant semantics)


def assert_close(y, r, atol=ATOL, rtol=RTOL, what=""):
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    err = np.abs(y - r)
    tol = atol + rtol * np.abs(r)
    bad = np.nonzero(~(err <= tol))[0]
    assert bad.size == 0, (f"{what}: {bad.size}/{r.size} outside |y-r| <= {atol} + {rtol}|r|; "
                           f"first {bad[:5].tolist()} y={y[bad[:5]].tolist()} r={r[bad[:5]].tolist()}")
    return float((err / tol).max()) if r.size else 0.0


def assert_bitwise(a, b, what=""):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    av, bv = a.view(np.uint8), b.view(np.uint8)
    if not np.array_equal(av, bv):
        if a.dtype == np.float32:
            d = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
            raise AssertionError(f"{what}: {d.size} elements differ, first {d[:5].tolist()} "
                                 f"{a[d[:5]].tolist()} vs {b[d[:5]].tolist()}")
        raise AssertionError(f"{what}: arrays differ")


def exact_weights_f64(dtype, w, n_rows, k):
    """The weights gemv_quant multiplies by, exactly, as float64 [n_rows, k]:
    Q4_K (d*sc)*q - dmin*m (quants.rs:151), Q6_K d*(sc*(raw-32)) (:195),
    Q8_0 d*q, each formed in f64 from the oracle's integer unpack (every
    intermediate is exact in f64). gemv_quant's output is the f32 rounding
    of sum(x_e * w_e) in f64, so X @ W.T in f64 differs from it only by the
    f64 summation order (a few 1e-16 relative; tests/test_oracle_kats.py
    checks this against the oracle itself)."""
    import oracle as O
    if dtype == O.Q4_K:
        q, sc, m, d, dmin = O.unpack_q4_k(w)
        q = q.reshape(-1, 8, 32).astype(np.float64)
        ds = d.astype(np.float64)[:, None] * sc.reshape(-1, 8).astype(np.float64)
        dm = dmin.astype(np.float64)[:, None] * m.reshape(-1, 8).astype(np.float64)
        W = ds[:, :, None] * q - dm[:, :, None]
    elif dtype == O.Q6_K:
        q, sc, d = O.unpack_q6_k(w)
        q = q.reshape(-1, 16, 16).astype(np.float64) - 32.0
        W = d.astype(np.float64)[:, None, None] * (sc.reshape(-1, 16).astype(np.float64)[:, :, None] * q)
    elif dtype == O.Q8_0:
        q, d = O.unpack_q8_0(w)
        W = d.astype(np.float64)[:, None] * q.reshape(-1, 32).astype(np.float64)
    else:
        raise ValueError(dtype)
    return W.reshape(n_rows, k)


def gemm_reference(dtype, w, n_rows, k, X):
    """Y[m] = gemv_quant(X[m]) for every row, through exact_weights_f64."""
    W = exact_weights_f64(dtype, w, n_rows, k)
    return (np.asarray(X, np.float32).astype(np.float64) @ W.T)


def swiglu_bound(rg, ru):
    """Bound on |h - swiglu(rg, ru)| when h = swiglu(g, u) of GEMV outputs g,
    u that each meet the gemv_quant tolerance around the reference rg, ru:
    the tolerance itself plus the reference tolerance propagated through
    silu'(g) u and silu(g)."""
    g64, u64 = np.asarray(rg, np.float64), np.asarray(ru, np.float64)
    sig = 1.0 / (1.0 + np.exp(-g64))
    rh = g64 * sig * u64
    dsilu = sig * (1.0 + g64 * (1.0 - sig))
    tol_g, tol_u = ATOL + RTOL * np.abs(g64), ATOL + RTOL * np.abs(u64)
    return rh, ATOL + RTOL * np.abs(rh) + np.abs(dsilu * u64) * tol_g + np.abs(g64 * sig) * tol_u
