"""CPU checks of uq_gemm_q8k's operand maps (uq_q8k_tiles.h) through the host
emulation (libuq_emu.so): the activation octets filled by the prep's slot
map, the weight octets decoded by the kernel's gathers and bit-field
inserts, the lane sums as the octets' slot products, the reference's f32
epilogue. Every row must equal the oracle's gemv_quant_q8k
(quants.rs:474-515) bit for bit, so a slot that pairs the wrong activation
and weight, a wrong byte, nibble, qh field or scale, or an epilogue out of
the reference's order fails here before the kernel runs on a GPU."""
import numpy as np
import pytest

import oracle as O
import uq
import uq.synth as S
from helpers import assert_bitwise


def _check(dtype, w, K, N, X):
    Y = uq.emu_gemm_q8k(X, w, K, N, dtype)
    for m in range(X.shape[0]):
        ref = np.zeros(N, np.float32)
        O.gemv_quant_q8k(ref, X[m], w, K, N, dtype)
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(Y[m]), nan), f"row {m}: NaN positions"
        assert_bitwise(Y[m][~nan], ref[~nan], f"dtype {dtype} row {m}")


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K])
@pytest.mark.parametrize("K,N,M", [(256, 16, 3), (1024, 24, 5), (2048, 9, 2)])
def test_emulated_gemm_q8k_equals_gemv_quant_q8k(dtype, K, N, M):
    w = S.weights(dtype, N, K, seed=K + N + dtype)
    X = S.activations(K, seed=M + K, rows=M).reshape(M, K)
    _check(dtype, w, K, N, X)


def test_emulated_gemm_q8k_q6k_full_int8_scales():
    """Q6_K scales over the whole int8 range, where sc*q needs the exact
    (sc & ~1)*q + (sc & 1)*q pair."""
    K, N, M = 512, 16, 3
    w = S.weights(S.Q6_K, N, K, seed=5).reshape(-1, 210)
    rng = np.random.default_rng(6)
    w[:, 192:208] = rng.integers(-128, 128, size=(w.shape[0], 16)).astype(np.int8).view(np.uint8)
    w[::3, 192:208] = np.uint8(0x80)  # -128 everywhere in some blocks
    X = S.activations(K, seed=7, rows=M).reshape(M, K)
    _check(S.Q6_K, w.reshape(-1), K, N, X)


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K])
def test_emulated_gemm_q8k_edge_rows(dtype):
    """A zero row, a zero block, a row whose maximum is negative, ties in
    |x|, a NaN (quantizes to 0) and an infinity (d = -inf: the row is NaN)."""
    K, N, M = 512, 12, 6
    X = S.activations(K, seed=3, rows=M).reshape(M, K).copy()
    X[0] = 0.0
    X[1, :256] = 0.0
    X[2, 100] = -50.0
    X[3, 10], X[3, 20] = 7.0, -7.0
    X[4, 33] = np.nan
    X[5, 300] = np.inf
    w = S.weights(dtype, N, K, seed=11)
    _check(dtype, w, K, N, X)
