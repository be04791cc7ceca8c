"""GPU parity of the prefill GEMM (uq_gemm) through the C ABI.

uq_gemm computes Y[m] = gemv_quant(W, X[m]) for every row (the reference
feeds prefill tokens one at a time, greedy.rs:55-65; quants.rs:422-466).
Bar: |y - r| <= 1e-4 + 1e-3 |r| per element, r the f64 sum of exact
products. At full size r comes from helpers.gemm_reference (the exact f64
weights of the oracle's integer unpack times X in f64, pinned against the
oracle's gemv_quant in tests/test_oracle_kats.py); a few rows of every case
are also compared with the oracle's gemv_quant itself.

The shapes cover each kernel shape the launcher picks (128 x 192 and 64 x 256
for Q4_K, 128 x 128 and 64 x 128 for Q6_K and Q8_0, and for M <= 32 the
loader-wave kernel of each format),
several 256-k blocks per workgroup (the LDS rings' steady state and the
per-block scaling), K split across workgroups (even and uneven ranges),
masked M and N tails, and the activation prep's three K regimes.
"""
import os
import sys

import numpy as np
import pytest

import oracle as O
import uq
import uq.synth as S
from helpers import assert_close, exact_weights_f64, gemm_reference

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def run_gemm(dtype, w, K, N, X):
    M = X.shape[0]
    W = uq.Weights(w, dtype, K, N)
    dx, dy = uq.DeviceArray.from_numpy(np.ascontiguousarray(X, np.float32)), uq.DeviceArray(4 * M * N)
    uq.gemm(W, M, dx, dy)
    Y = dy.download(np.float32, M * N).reshape(M, N)
    W.free()
    return Y


def check_rows(dtype, w, K, N, X, Y, what, oracle_rows=3):
    R = gemm_reference(dtype, w, N, K, X)
    worst = 0.0
    for m in range(X.shape[0]):
        worst = max(worst, assert_close(Y[m], R[m], what=f"{what} row {m}"))
    for m in sorted({0, X.shape[0] - 1, X.shape[0] // 2})[:oracle_rows]:
        ref = np.zeros(N, np.float32)
        O.gemv_quant(ref, X[m], w, K, N, dtype, nthreads=NT)
        assert_close(Y[m], ref, what=f"{what} row {m} vs oracle gemv_quant")
    return worst


@pytest.mark.parametrize("K,N,M", [(4096, 12288, 512), (4096, 12288, 128), (4096, 6144, 200)])
def test_gemm_q4k_prefill_config(K, N, M):
    """The prefill workload itself (Q4_K 12288 x 4096, M = 512 and 128) and
    an uneven one: 16 blocks per workgroup at M = 512, K split into ranges
    of several blocks at M = 128 and 200."""
    log(f"gemm q4k K={K} N={N} M={M}")
    w = S.weights(S.Q4_K, N, K, seed=S.seed_for(3))
    X = S.activations(K, seed=S.seed_for(3) + M, rows=M).reshape(M, K)
    worst = check_rows(S.Q4_K, w, K, N, X, run_gemm(S.Q4_K, w, K, N, X), f"q4k {M}x{N}x{K}")
    log(f"worst err/tol {worst:.3g}")


Q4K_SHAPES = [
    # M <= 32 (the loader-wave kernel, 256 columns per workgroup), split K (ranges of one to four
    # blocks; two at 2560 x 12288); one to seven rows
    (4096, 1024, 1), (4096, 1024, 2), (4096, 1024, 3), (4096, 768, 5), (4096, 1000, 7), (4096, 12288, 8),
    (12288, 600, 16), (768, 512, 32), (2560, 12288, 4),
    # 64 x 256 tiles (32 < M <= 64)
    (4096, 256, 33), (5120, 200, 40), (1280, 1000, 64),
    # 128 x 192 tiles (M > 64): one block, a few blocks, many; tails in M and N
    (256, 768, 257), (512, 384, 70), (1024, 600, 400), (4096, 3072, 96), (16640, 192, 80),
    (12288, 4096, 130),
]


@pytest.mark.parametrize("K,N,M", Q4K_SHAPES)
def test_gemm_q4k_shapes(K, N, M):
    log(f"gemm q4k K={K} N={N} M={M}")
    w = S.weights(S.Q4_K, N, K, seed=N + M)
    X = S.activations(K, seed=K + M, rows=M).reshape(M, K)
    check_rows(S.Q4_K, w, K, N, X, run_gemm(S.Q4_K, w, K, N, X), f"q4k {M}x{N}x{K}")


@pytest.mark.parametrize("dtype", [S.Q6_K, S.Q8_0])
@pytest.mark.parametrize("K,N,M", [(4096, 12288, 512), (12288, 4096, 300), (12288, 4096, 100), (12288, 4096, 8),
                                   (4096, 12288, 8), (4096, 12288, 20), (4096, 1000, 70),
                                   (256, 200, 3), (1024, 130, 65), (4352, 384, 33), (12288, 1000, 29)])
def test_gemm_q6k_q8_0(dtype, K, N, M):
    """Q6_K and Q8_0 on the MFMA: the prefill shape (N = 12288, K = 4096,
    M = 512; Q8_0 on 256 x 96 tiles), the down-projection shape (K = 12288)
    at M = 300, 100 and 8, and small / ragged shapes (M <= 32 runs the
    loader-wave kernels: 128- or 96-column workgroups, 96 at N = 12288 and
    K = 4096 for M = 8 and 20, tiles past N, K split into ranges of one or
    two blocks at 12288 x 1000)."""
    log(f"gemm dtype={dtype} K={K} N={N} M={M}")
    w = S.weights(dtype, N, K, seed=K + N + M + dtype)
    X = S.activations(K, seed=M + dtype, rows=M).reshape(M, K)
    check_rows(dtype, w, K, N, X, run_gemm(dtype, w, K, N, X), f"dtype {dtype} {M}x{N}x{K}")


def test_gemm_q6k_full_int8_scales():
    """Q6_K scales over the whole int8 range (real files reach -128): the
    weight splits (sc & ~1)*q + (sc & 1)*q stay exact where sc*q alone would
    not fit an f16 integer."""
    K, N, M = 2048, 512, 80
    w = S.weights(S.Q6_K, N, K, seed=5).reshape(-1, 210)
    rng = np.random.default_rng(6)
    w[:, 192:208] = rng.integers(-128, 128, size=(w.shape[0], 16)).astype(np.int8).view(np.uint8)
    w[::7, 192] = np.uint8(0x80)  # -128
    w = w.reshape(-1)
    X = S.activations(K, seed=7, rows=M).reshape(M, K)
    check_rows(S.Q6_K, w, K, N, X, run_gemm(S.Q6_K, w, K, N, X), "q6k int8 scales")


# Outputs of test_gemm_dynamic_range that need the accumulation term (miss
# 1e-4 + 1e-3|r| alone), per (format, M); every other case has none.
STRICT_MISSES = {(S.Q6_K, 70): 1}


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K, S.Q8_0])
@pytest.mark.parametrize("M", [70, 12])
def test_gemm_dynamic_range(dtype, M):
    """Rows of very different magnitude (1e-4 .. 1e4), rows spanning many
    binades, a zero row, a row with one large entry and rows of tiny or
    subnormal values: the per-row
    power-of-two scale and the f16 hi/lo split keep the operands exact to
    22 bits. The matrix cores accumulate in f32, so an output whose terms
    cancel deeply sits within the gemv_quant tolerance plus the accumulation
    term 2^-22 * sum_e |x_e w_e| (the GEMM's stated bound; at these row
    magnitudes, 1e-4 alone would ask for 2^-26 of the terms' sum)."""
    K, N = 1024, 256
    rng = np.random.default_rng(11)
    X = rng.standard_normal((M, K)).astype(np.float32)
    X *= (10.0 ** rng.uniform(-4, 4, size=(M, 1))).astype(np.float32)
    X[::3] *= (10.0 ** rng.uniform(-6, 0, size=(len(X[::3]), K))).astype(np.float32)
    X[5] = 0.0
    X[7, :] = 0.0
    X[7, 100] = 3.0e4
    # rows near the bottom of the f32 range (max|x| ~ 2^-124, and subnormals):
    # the row exponent is clamped so that 1/s stays finite
    X[9] = (rng.standard_normal(K) * 1e-38).astype(np.float32)
    X[11] = (rng.standard_normal(K) * 1e-41).astype(np.float32)
    w = S.weights(dtype, N, K, seed=99)
    Y = run_gemm(dtype, w, K, N, X)
    Wx = exact_weights_f64(dtype, w, N, K)
    R = X.astype(np.float64) @ Wx.T
    A = np.abs(X.astype(np.float64)) @ np.abs(Wx).T  # sum_e |x_e w_e|
    err = np.abs(Y.astype(np.float64) - R)
    bound = 1e-4 + 1e-3 * np.abs(R) + 2.0 ** -22 * A
    bad = np.argwhere(~(err <= bound))
    assert bad.size == 0, f"{len(bad)} outside the bound, first {bad[:3].tolist()}"
    strict = np.argwhere(~(err <= 1e-4 + 1e-3 * np.abs(R)))
    log(f"dtype {dtype}: {len(strict)} of {err.size} outputs need the accumulation term; "
        f"worst err / sum|xw| = {float(np.max(err / np.maximum(A, 1e-300))):.3g}")
    # every other output meets the strict gemv_quant bound: the exact count
    # measured on these inputs (the kernels are deterministic) is the ceiling
    ceiling = STRICT_MISSES.get((dtype, M), 0)
    assert len(strict) <= ceiling, f"{len(strict)} outputs outside 1e-4 + 1e-3|r| (ceiling {ceiling})"


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K, S.Q8_0])
def test_gemm_split_k_cancellation_bound(dtype):
    """Small M at K = 12288 on a narrow N, so K is split across 24-48
    workgroups per column group, with rows built to cancel: row m is a random
    vector with its projection on weight rows 7m .. 7m + 6 removed, so those
    outputs are tiny against sum_e |x_e w_e|. The partial tiles stay f64 and
    are summed in range order, so the split adds nothing to the stated bound
    1e-4 + 1e-3 |r| + 2^-22 sum_e |x_e w_e|."""
    K, N, M = 12288, 1000, 8
    w = S.weights(dtype, N, K, seed=77 + dtype)
    Wx = exact_weights_f64(dtype, w, N, K)
    rng = np.random.default_rng(78)
    X = np.empty((M, K), np.float32)
    for m in range(M):
        z = rng.standard_normal(K) * 100.0
        Q, _ = np.linalg.qr(Wx[7 * m:7 * m + 7].T)
        X[m] = (z - Q @ (Q.T @ z)).astype(np.float32)
    Y = run_gemm(dtype, w, K, N, X)
    R = X.astype(np.float64) @ Wx.T
    A = np.abs(X.astype(np.float64)) @ np.abs(Wx).T
    err = np.abs(Y.astype(np.float64) - R)
    bad = np.argwhere(~(err <= 1e-4 + 1e-3 * np.abs(R) + 2.0 ** -22 * A))
    assert bad.size == 0, f"{len(bad)} outside the bound, first {bad[:3].tolist()}"
    planted = np.array([[m, 7 * m + j] for m in range(M) for j in range(7)])
    ratio = np.abs(R[planted[:, 0], planted[:, 1]]) / A[planted[:, 0], planted[:, 1]]
    assert np.all(ratio < 1e-6), "the planted outputs cancel"
    strict = np.argwhere(~(err <= 1e-4 + 1e-3 * np.abs(R)))
    log(f"dtype {dtype}: {len(strict)} of {err.size} outputs need the accumulation term; "
        f"worst err / sum|xw| = {float(np.max(err / A)):.3g}")


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K, S.Q8_0])
def test_gemm_non_finite_rows_are_nan(dtype):
    """A row holding a NaN or an infinity gives NaN outputs (gemv_quant's f64
    sum is NaN, or +-inf by the row's weights, for such a row: non-finite
    either way); every other row is unaffected."""
    K, N, M = 1024, 300, 40
    X = S.activations(K, seed=13, rows=M).reshape(M, K)
    X[3, 17] = np.nan
    X[20, 1000] = np.inf
    X[21, 0] = -np.inf
    w = S.weights(dtype, N, K, seed=14)
    Y = run_gemm(dtype, w, K, N, X)
    bad = [3, 20, 21]
    assert np.all(np.isnan(Y[bad])), "non-finite rows"
    good = [m for m in range(M) if m not in bad]
    R = gemm_reference(dtype, w, N, K, X[good])
    for i, m in enumerate(good):
        assert_close(Y[m], R[i], what=f"finite row {m}")


def test_gemm_dim_in_zero_writes_zeros():
    """dim_in == 0: every output is the empty dot, 0 (gemv_quant's pairwise
    sum of nothing); no activation is read."""
    N, M = 100, 9
    W = uq.Weights(np.zeros(0, np.uint8), S.Q4_K, 0, N)
    dx, dy = uq.DeviceArray(16), uq.DeviceArray(4 * M * N)
    dy.upload(np.full(M * N, 7.0, np.float32))
    uq.gemm(W, M, dx, dy)
    assert np.all(dy.download(np.float32, M * N) == 0.0)


def test_gemm_is_deterministic_and_regrows_its_workspace():
    """Repeat calls give the same bits (split-K partials are summed in range
    order); a call with a larger M grows the workspace, a smaller one after
    it reuses it, and results stay within tolerance."""
    K, N = 2048, 1000
    w = S.weights(S.Q4_K, N, K, seed=7)
    W = uq.Weights(w, S.Q4_K, K, N)
    for M in (24, 24, 300, 5):
        X = S.activations(K, seed=M, rows=M).reshape(M, K)
        dx = uq.DeviceArray.from_numpy(X)
        outs = []
        for _ in range(2):
            dy = uq.DeviceArray(4 * M * N)
            uq.gemm(W, M, dx, dy)
            outs.append(dy.download(np.float32, M * N))
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), f"M={M}"
        R = gemm_reference(S.Q4_K, w, N, K, X)
        for m in range(M):
            assert_close(outs[0].reshape(M, N)[m], R[m], what=f"M={M} row {m}")
