"""The kernels' per-lane code, run on the CPU (libuq_emu.so), against the oracle.

The emulation compiles the same policy code the gfx950 kernels run
(unltd-inference_amd/csrc/uq_policies.h) for the host, with the workgroup
activation prep, wave row loop, DPP reduction tree and Q8_K epilogue written
as loops. Shapes cover every fast-path branch: one block, partial waves,
K = 4096 (one task per lane, VGPR-cached activations), K = 12288 (three tasks
per lane, LDS-streamed), 2-byte-aligned Q6_K/Q8_0 blocks.
"""
import numpy as np
import pytest

import oracle as O
import uq
import uq.synth as S
from helpers import assert_bitwise, assert_close

SHAPES = [(256, 7), (512, 3), (1024, 9), (4096, 33), (8192, 5), (12288, 9)]


@pytest.mark.parametrize("dtype", [O.Q4_K, O.Q6_K, O.Q8_0])
@pytest.mark.parametrize("K,N", SHAPES)
def test_emulated_gemv_matches_gemv_quant(dtype, K, N):
    w = S.weights(dtype, N, K, seed=1000 + K + N + dtype)
    x = S.activations(K, seed=K + dtype)
    ref = np.zeros(N, np.float32)
    O.gemv_quant(ref, x, w, K, N, dtype, nthreads=4)
    assert_close(uq.emu_gemv(x, w, K, N, dtype), ref, what=f"dtype {dtype} K {K}")


@pytest.mark.parametrize("dtype", [O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("K,N", SHAPES)
def test_emulated_gemv_q8k_is_bit_exact(dtype, K, N):
    w = S.weights(dtype, N, K, seed=2000 + K + N + dtype)
    x = S.activations(K, seed=7 * K + dtype)
    ref = np.zeros(N, np.float32)
    O.gemv_quant_q8k(ref, x, w, K, N, dtype, nthreads=4)
    assert_bitwise(uq.emu_gemv(x, w, K, N, dtype, q8k=True), ref, what=f"q8k dtype {dtype} K {K}")


@pytest.mark.parametrize("dtype", [O.Q4_K, O.Q6_K, O.Q8_0])
def test_emulated_gemv_activation_edge_cases(dtype):
    """Zero runs, a huge outlier per run, tiny and subnormal values, sign
    flips: the fixed-point activation form must stay within tolerance."""
    K, N = 4096, 17
    w = S.weights(dtype, N, K, seed=77)
    rng = np.random.default_rng(5)
    x = rng.standard_normal(K).astype(np.float32)
    x[0:32] = 0.0
    x[64:96] *= 1e-30
    x[96] = 3e4
    x[200:232] = np.float32(1e-41)  # subnormal f32
    x[512:1024] *= -1e3
    ref = np.zeros(N, np.float32)
    O.gemv_quant(ref, x, w, K, N, dtype)
    assert_close(uq.emu_gemv(x, w, K, N, dtype), ref, what="edge activations")


@pytest.mark.parametrize("dtype", [O.Q4_K, O.Q6_K])
def test_emulated_q8k_edge_cases(dtype):
    """Zero blocks, ties for max |x|, negative max, all-equal blocks."""
    K, N = 1024, 11
    w = S.weights(dtype, N, K, seed=78)
    x = S.activations(K, seed=9)
    x[0:256] = 0.0
    x[256:512] = -1.0
    x[600], x[601] = 7.0, -7.0
    x[900] = -9.5
    ref = np.zeros(N, np.float32)
    O.gemv_quant_q8k(ref, x, w, K, N, dtype)
    assert_bitwise(uq.emu_gemv(x, w, K, N, dtype, q8k=True), ref, what="q8k edges")


def test_emulated_reference_pins():
    """The four real GGUF blocks of the reference pins through the kernel
    code (quants.rs:1154-1222, gguf-py values, tolerance 1e-4)."""
    import json, os
    fx = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_pins.json")))
    i = np.arange(256)
    xp = ((i * 7919) % 1009).astype(np.float32) / np.float32(1009.0) - np.float32(0.5)
    xa = ((i * 31 + 17) % 257).astype(np.float32) / np.float32(257.0) - np.float32(0.5)
    for case in fx["cases"]:
        blk = np.frombuffer(bytes(fx["blocks"][case["block"]]["bytes"]), np.uint8)
        dt = O.Q6_K if blk.size == 210 else O.Q4_K
        for x, key in ((xp, "dot_x_pattern"), (xa, "dot_x_alt")):
            y = uq.emu_gemv(x, blk, 256, 1, dt)
            assert abs(float(y[0]) - case[key]) < fx["tolerance"], (case["block"], key)


@pytest.mark.parametrize("dtype", [O.Q4_K, O.Q6_K, O.Q8_0])
@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_emulated_gemv_non_finite_activation_gives_nan(dtype, bad):
    """A NaN or infinite activation makes its run's scale NaN, so every row
    is NaN; gemv_quant gives NaN (NaN input) or +-inf / NaN (infinite input)
    for such rows: non-finite either way, never a finite number."""
    K, N = 1024, 9
    w = S.weights(dtype, N, K, seed=79)
    x = S.activations(K, seed=10)
    x[517] = bad
    ref = np.zeros(N, np.float32)
    O.gemv_quant(ref, x, w, K, N, dtype)
    assert not np.any(np.isfinite(ref))
    y = uq.emu_gemv(x, w, K, N, dtype)
    assert np.all(np.isnan(y)), y
