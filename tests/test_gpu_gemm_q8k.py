"""GPU parity of uq_gemm_q8k through the C ABI: Y[m] = gemv_quant_q8k(W, X[m])
(quants.rs:474-515) for every row, bit for bit against the oracle.

The reference forward prefills token by token through gemv_quant_q8k
(greedy.rs:55-65; qwen35_forward.rs:365-401), so every row of the batched
call must carry exactly the bits of that token's call. The shapes cover the
prefill workload itself (Q4_K 12288 x 4096 at M = 512), the Q6_K FFN-down
shape (4096 x 12288), each tile the launcher picks (64-row waves in
eight-wave workgroups for M > 128, 32-row waves in six, two or one-wave
workgroups, 16-row waves for M <= 16), ragged M (padding rows) and N
(columns past the end), one block, many blocks, and the edge cases of the
quantizer and of the block scales.
"""
import os
import sys

import numpy as np
import pytest

import oracle as O
import uq
import uq.synth as S
from helpers import assert_bitwise

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def run(dtype, w, K, N, X):
    M = X.shape[0]
    W = uq.Weights(w, dtype, K, N)
    dx, dy = uq.DeviceArray.from_numpy(np.ascontiguousarray(X, np.float32)), uq.DeviceArray(4 * M * N)
    dy.upload(np.full(M * N, np.nan, np.float32))
    uq.gemm_q8k(W, M, dx, dy)
    Y = dy.download(np.float32, M * N).reshape(M, N)
    W.free()
    return Y


def oracle_rows(dtype, w, K, N, X, rows=None):
    rows = range(X.shape[0]) if rows is None else rows
    out = {}
    for m in rows:
        r = np.zeros(N, np.float32)
        O.gemv_quant_q8k(r, X[m], w, K, N, dtype, nthreads=NT)
        out[m] = r
    return out


def assert_rows(Y, R, what):
    for m, r in R.items():
        nan = np.isnan(r)
        assert np.array_equal(np.isnan(Y[m]), nan), f"{what} row {m}: NaN positions differ"
        assert_bitwise(Y[m][~nan], r[~nan], f"{what} row {m}")


def test_gemm_q8k_prefill_config_every_row():
    """The prefill workload: Q4_K N = 12288, K = 4096, M = 512 (64 x 128
    workgroup tiles, 16 blocks each), every row against the oracle."""
    K, N, M = 4096, 12288, 512
    log(f"gemm_q8k q4k K={K} N={N} M={M}")
    w = S.weights(S.Q4_K, N, K, seed=S.seed_for(3))
    X = S.activations(K, seed=S.seed_for(3) + M, rows=M).reshape(M, K)
    Y = run(S.Q4_K, w, K, N, X)
    assert_rows(Y, oracle_rows(S.Q4_K, w, K, N, X), "q4k prefill")


def test_gemm_q8k_q6k_down_shape_every_row():
    """Q6_K N = 4096, K = 12288 (an FFN down projection), M = 300: 48 blocks
    per row, ragged M (the last tile's padding rows), every row."""
    K, N, M = 12288, 4096, 300
    log(f"gemm_q8k q6k K={K} N={N} M={M}")
    w = S.weights(S.Q6_K, N, K, seed=S.seed_for(2))
    X = S.activations(K, seed=M + 1, rows=M).reshape(M, K)
    Y = run(S.Q6_K, w, K, N, X)
    assert_rows(Y, oracle_rows(S.Q6_K, w, K, N, X), "q6k down")


SHAPES = [
    # (K, N, M): 16-row tiles for M <= 16 (one wave per workgroup at these
    # N) and where 32 x 64 tiles would number under one per CU (M = 64 at
    # N = 4096: four waves a workgroup; M = 128 at N = 1024: two); 32-row
    # tiles of four waves (M = 64, 100, 128 at N >= 4096); 64-row tiles past
    # M = 128 where they fill the CUs (M = 200 at N = 8192). The K-parallel
    # kernel where 16 x 16 tiles number at most one per CU and K >= 2048 (M =
    # 31, 33, 65, M = 8 at K = 12288, the 32-wide projections of a 512- or
    # 300-token prefill), and for M <= 32 at K > 8192 up to two per CU (M =
    # 24 at K = 12288)
    (256, 300, 2), (768, 1000, 3), (1024, 256, 8), (4096, 2048, 31), (2048, 777, 33),
    (4096, 12288, 64), (4096, 12288, 128), (1280, 4096, 100), (512, 8192, 200), (4096, 640, 65),
    (12288, 4096, 8), (2304, 48, 16), (12288, 4096, 24), (4096, 32, 512), (4096, 40, 300), (12288, 4096, 100),
    (4096, 4096, 64), (4096, 1024, 128),
]


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K])
@pytest.mark.parametrize("K,N,M", SHAPES)
def test_gemm_q8k_shapes(dtype, K, N, M):
    log(f"gemm_q8k dtype={dtype} K={K} N={N} M={M}")
    w = S.weights(dtype, N, K, seed=K + N + M + dtype)
    X = S.activations(K, seed=M * 7 + dtype, rows=M).reshape(M, K)
    Y = run(dtype, w, K, N, X)
    rows = sorted({0, 1, M // 2, M - 1} | set(range(0, M, max(1, M // 12))))
    assert_rows(Y, oracle_rows(dtype, w, K, N, X, rows), f"dtype {dtype} {M}x{N}x{K}")


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K])
def test_gemm_q8k_equals_per_row_gemv_q8k(dtype):
    """Every row equals the device's own gemv_quant_q8k of that row (the
    decode kernel, checked against the oracle elsewhere), at a shape with
    several tiles in both directions."""
    K, N, M = 2048, 1536, 70
    w = S.weights(dtype, N, K, seed=21 + dtype)
    X = S.activations(K, seed=22, rows=M).reshape(M, K)
    Y = run(dtype, w, K, N, X)
    W = uq.Weights(w, dtype, K, N)
    for m in range(M):
        dx, dy = uq.DeviceArray.from_numpy(X[m]), uq.DeviceArray(4 * N)
        uq.gemv_q8k(W, dx, dy)
        assert_bitwise(Y[m], dy.download(np.float32, N), f"row {m} vs gemv_q8k")
    W.free()


def test_gemm_q8k_q6k_full_int8_scales():
    """Q6_K scales over the whole int8 range (real files reach -128): the
    exact (sc & ~1)*q + (sc & 1)*q operand pair."""
    K, N, M = 2048, 512, 80
    w = S.weights(S.Q6_K, N, K, seed=5).reshape(-1, 210)
    rng = np.random.default_rng(6)
    w[:, 192:208] = rng.integers(-128, 128, size=(w.shape[0], 16)).astype(np.int8).view(np.uint8)
    w[::7, 192:208] = np.uint8(0x80)
    w = w.reshape(-1)
    X = S.activations(K, seed=7, rows=M).reshape(M, K)
    Y = run(S.Q6_K, w, K, N, X)
    assert_rows(Y, oracle_rows(S.Q6_K, w, K, N, X), "q6k int8 scales")


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K])
def test_gemm_q8k_special_block_scales(dtype):
    """Blocks whose f16 d (and Q4_K dmin) is subnormal, the largest finite,
    zero, negative, infinite or NaN (f16_to_f32, quants.rs:44-72): numbers
    bit for bit, NaN where the reference is NaN."""
    K, N, M = 1024, 96, 40
    w = S.weights(dtype, N, K, seed=K + N + dtype).reshape(N, -1)
    bb = 144 if dtype == S.Q4_K else 210
    doff = 0 if dtype == S.Q4_K else 208
    specials = [0x0001, 0x03FF, 0x0200, 0x7BFF, 0x0000, 0x8000, 0x83FF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0x7D01]
    rng = np.random.default_rng(dtype + K)
    for r in range(N):
        blk = int(rng.integers(0, K // 256))
        v = specials[r % len(specials)]
        w[r, blk * bb + doff] = v & 0xFF
        w[r, blk * bb + doff + 1] = v >> 8
        if dtype == S.Q4_K and r % 3 == 0:
            v2 = specials[(r // 3) % len(specials)]
            w[r, blk * bb + 2] = v2 & 0xFF
            w[r, blk * bb + 3] = v2 >> 8
    w = w.reshape(-1)
    X = S.activations(K, seed=N + 5, rows=M).reshape(M, K)
    Y = run(dtype, w, K, N, X)
    R = oracle_rows(dtype, w, K, N, X)
    assert any(np.isnan(r).any() for r in R.values()), "the test plants infinite and NaN scales"
    assert_rows(Y, R, f"special scales dtype {dtype}")


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K])
def test_gemm_q8k_edge_activations(dtype):
    """Rows of the quantizer's edge cases: zero rows and blocks, a negative
    maximum, ties in |x| (within a lane's four elements and across lanes of
    one block, either sign first), subnormals, rows of very different magnitude, a
    NaN (quantized to 0: the row stays finite) and an infinity (d = -inf:
    the row is NaN in the reference and here)."""
    K, N, M = 1024, 200, 36
    rng = np.random.default_rng(dtype)
    X = S.activations(K, seed=9, rows=M).reshape(M, K).copy()
    X *= (10.0 ** rng.uniform(-6, 6, size=(M, 1))).astype(np.float32)
    X[0] = 0.0
    X[1, 256:512] = 0.0
    X[2, 700] = -1e5
    X[3, 5], X[3, 6] = 3.0e3, -3.0e3
    X[4] = (rng.standard_normal(K) * 1e-41).astype(np.float32)
    X[5, 17] = np.nan
    X[6, 600] = np.inf
    X[7, 1] = -np.inf
    X[8, 10], X[8, 100] = -5.0e3, 5.0e3
    X[9, 40], X[9, 200] = -7.0e3, 7.0e3
    X[10, 300], X[10, 301], X[10, 509] = 9.0e3, -9.0e3, -9.0e3
    w = S.weights(dtype, N, K, seed=31 + dtype)
    Y = run(dtype, w, K, N, X)
    R = oracle_rows(dtype, w, K, N, X)
    assert np.all(np.isfinite(R[5])) and np.all(np.isnan(R[6]))
    assert_rows(Y, R, f"edge activations dtype {dtype}")


def test_gemm_q8k_one_row_is_gemv_q8k_and_errors():
    """m_rows == 1 runs the decode kernel (the same bits); Q8_0 and F32
    weights are refused as gemv_quant_q8k panics (quants.rs:497-499)."""
    K, N = 4096, 500
    w = S.weights(S.Q4_K, N, K, seed=3)
    X = S.activations(K, seed=4, rows=1).reshape(1, K)
    Y = run(S.Q4_K, w, K, N, X)
    assert_rows(Y, oracle_rows(S.Q4_K, w, K, N, X), "one row")
    W = uq.Weights(S.weights(S.Q8_0, 64, 256, seed=1), S.Q8_0, 256, 64)
    dx, dy = uq.DeviceArray(4 * 2 * 256), uq.DeviceArray(4 * 2 * 64)
    with pytest.raises(uq.UqError) as e:
        uq.gemm_q8k(W, 2, dx, dy)
    assert e.value.kind == "DTYPE"
    W.free()


BATCH_CASES = [
    # (K, segment widths, M): the GatedDeltaNet projections (qkv, z, beta,
    # alpha) at 128 tokens (32-row tiles of four waves) and 512 (64 x 128
    # tiles for qkv and z, the K-parallel kernel for the two 32-wide ones);
    # ragged widths over and under 128 columns at 200 rows; widths that end
    # inside a tile in every segment, at 37 rows; a
    # zero-width segment; two 32-wide segments on the K-parallel kernel (128
    # and 300 rows); M = 16 (16-row tiles); M = 1 (the batched decode
    # kernel); one segment
    (4096, (8192, 4096, 32, 32), 128),
    (4096, (8192, 4096, 32, 32), 512),
    (1024, (300, 100, 1100, 17), 200),
    (2048, (1000, 17, 300, 65), 37),
    (1024, (48, 0, 200), 70),
    (4096, (32, 32), 128),
    (4096, (32, 32), 300),
    (1536, (640, 96, 33), 16),
    (1024, (777, 40, 5), 1),
    (256, (300,), 2),
]


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K])
@pytest.mark.parametrize("K,widths,M", BATCH_CASES)
def test_gemm_q8k_batch_equals_each_gemm(dtype, K, widths, M):
    """uq_gemm_q8k_batch: one launch over every weight's column tiles; each
    output equals uq_gemm_q8k of its weight alone, bit for bit, and no
    output is written past its own columns."""
    log(f"gemm_q8k_batch dtype={dtype} K={K} widths={widths} M={M}")
    X = S.activations(K, seed=M * 3 + dtype, rows=M).reshape(M, K)
    dx = uq.DeviceArray.from_numpy(np.ascontiguousarray(X, np.float32))
    Ws, ys = [], []
    for i, N in enumerate(widths):
        Ws.append(uq.Weights(S.weights(dtype, N, K, seed=K + 31 * i + N + dtype), dtype, K, N))
        y = uq.DeviceArray(4 * (M * N + 64))  # 64 guard floats past each output
        y.upload(np.full(M * N + 64, np.nan, np.float32))
        ys.append(y)
    uq.gemm_q8k_batch(Ws, M, dx, ys)
    for i, (W, N) in enumerate(zip(Ws, widths)):
        got = ys[i].download(np.float32, M * N + 64)
        assert np.all(np.isnan(got[M * N:])), f"segment {i}: written past its outputs"
        ref = uq.DeviceArray(4 * max(M * N, 1))
        uq.gemm_q8k(W, M, dx, ref)
        want = ref.download(np.float32, M * N)
        assert not np.isnan(want).any()
        assert_bitwise(got[:M * N], want, f"segment {i} ({N} columns)")
        W.free()


def test_gemm_q8k_batch_rows_against_the_oracle():
    """Rows of a three-segment launch against the oracle's gemv_quant_q8k."""
    K, widths, M = 2048, (700, 40, 129), 50
    X = S.activations(K, seed=77, rows=M).reshape(M, K)
    dx = uq.DeviceArray.from_numpy(np.ascontiguousarray(X, np.float32))
    ws = [S.weights(S.Q4_K, N, K, seed=80 + N) for N in widths]
    Ws = [uq.Weights(w, S.Q4_K, K, N) for w, N in zip(ws, widths)]
    ys = [uq.DeviceArray(4 * M * N) for N in widths]
    uq.gemm_q8k_batch(Ws, M, dx, ys)
    for w, N, y in zip(ws, widths, ys):
        Y = y.download(np.float32, M * N).reshape(M, N)
        assert_rows(Y, oracle_rows(S.Q4_K, w, K, N, X, [0, 17, M - 1]), f"batch segment of {N}")
    for W in Ws:
        W.free()


def test_gemm_q8k_batch_errors():
    """More than four weights, or weights that differ in dtype or dim_in, are
    refused before anything is launched; Q8_0 is refused as in uq_gemm_q8k."""
    K = 512
    a = uq.Weights(S.weights(S.Q4_K, 64, K, seed=1), S.Q4_K, K, 64)
    b = uq.Weights(S.weights(S.Q6_K, 64, K, seed=2), S.Q6_K, K, 64)
    c = uq.Weights(S.weights(S.Q4_K, 64, 2 * K, seed=3), S.Q4_K, 2 * K, 64)
    q = uq.Weights(S.weights(S.Q8_0, 64, K, seed=4), S.Q8_0, K, 64)
    dx, dy = uq.DeviceArray(4 * 4 * 2 * K), uq.DeviceArray(4 * 4 * 64)
    for ws, kind in (([a] * 5, "ARG"), ([a, b], "LEN"), ([a, c], "LEN"), ([q], "DTYPE")):
        with pytest.raises(uq.UqError) as e:
            uq.gemm_q8k_batch(ws, 4, dx, [dy] * len(ws))
        assert e.value.kind == kind
    for W in (a, b, c, q):
        W.free()
