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
