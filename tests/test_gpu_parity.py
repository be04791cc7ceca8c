"""GPU parity: libuq's HIP kernels (through the C ABI) against the oracle.

Bars:
  * bit-exact: integer unpack, f32 dequantization, f16 decode, Q8_K
    quantization, gemv_quant_q8k;
  * gemv_quant semantics (GEMV, fused FFN, GEMM): |y - r| <= 1e-4 + 1e-3 |r|
    against the oracle's f64-accumulated gemv_quant;
  * and, as a diagnostic of the kernel plumbing, the device result of the
    fast GEMV kernels equals the CPU emulation of their per-lane code bit
    for bit.
Full-size shapes (152064 x 4096 Q6_K head, 12288 x 4096 FFN) are compared
row for row against the (multi-threaded) oracle.
"""
import json
import os
import sys

import numpy as np
import pytest

import oracle as O
import uq
import uq.synth as S
from helpers import assert_bitwise, assert_close

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# --------------------------------------------------------------- block level

def test_device_is_gfx950():
    assert uq.device_count() >= 1
    name = uq.device_name()
    log("device:", name)
    assert "gfx950" in name


def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    got = uq.f16_to_f32(h)
    ref = O.f16_to_f32_array(h)
    assert_bitwise(got, ref, "f16_to_f32")


def test_hardware_f16_conversion_in_gemv_matches_reference_decode():
    """The hot kernels convert block scales with v_cvt_f32_f16. Q8_0 rows
    whose first (or second) block has d = every f16 pattern, q = (1, 0, ...),
    x = e_0 (+ e_32): y must equal f16_to_f32 of the pattern exactly (the
    fixed-point activation of 1.0 is exact). NaN patterns excluded."""
    pats = np.arange(65536, dtype=np.uint16)
    pats = pats[~(((pats >> 10) & 0x1F) == 0x1F) | ((pats & 0x3FF) == 0)]  # drop NaNs
    n = pats.size
    w = np.zeros((2 * n, 68), np.uint8)
    pb = pats.view(np.uint8).reshape(n, 2)
    w[:n, 0:2] = pb
    w[:n, 2] = 1
    w[n:, 34:36] = pb
    w[n:, 36] = 1
    x = np.zeros(64, np.float32)
    x[0] = x[32] = 1.0
    y = np.zeros(2 * n, np.float32)
    uq.gemv_quant(y, x, w.reshape(-1), 64, 2 * n, uq.DType.Q8_0)
    # the row sum adds +0.0 from the other lanes, so -0.0 comes out as +0.0
    # (as the reference's pairwise sum would); compare with zeros canonical
    ref = O.f16_to_f32_array(pats) + np.float32(0.0)
    assert_bitwise(y[:n] + np.float32(0.0), ref, "cvt lo half")
    assert_bitwise(y[n:] + np.float32(0.0), ref, "cvt hi half")


@pytest.mark.parametrize("nblocks", [1, 37, 4096])
def test_unpack_q4_k_bit_exact(nblocks):
    w = S.blocks(S.Q4_K, nblocks, np.random.default_rng(nblocks))
    for got, ref, what in zip(uq.unpack_q4_k(w), O.unpack_q4_k(w), ("q", "sc", "m", "d", "dmin")):
        assert_bitwise(got, ref, f"unpack_q4_k {what}")


@pytest.mark.parametrize("nblocks", [1, 37, 4096])
def test_unpack_q6_k_bit_exact(nblocks):
    w = S.blocks(S.Q6_K, nblocks, np.random.default_rng(nblocks + 1))
    for got, ref, what in zip(uq.unpack_q6_k(w), O.unpack_q6_k(w), ("q", "sc", "d")):
        assert_bitwise(got, ref, f"unpack_q6_k {what}")


@pytest.mark.parametrize("nblocks", [1, 37, 4096])
def test_unpack_q8_0_bit_exact(nblocks):
    w = S.blocks(S.Q8_0, nblocks, np.random.default_rng(nblocks + 2))
    for got, ref, what in zip(uq.unpack_q8_0(w), O.unpack_q8_0(w), ("q", "d")):
        assert_bitwise(got, ref, f"unpack_q8_0 {what}")


@pytest.mark.parametrize("dtype,fn_uq,fn_or", [
    (S.Q4_K, uq.dequantize_q4_k, O.dequantize_q4_k),
    (S.Q6_K, uq.dequantize_q6_k, O.dequantize_q6_k),
    (S.Q8_0, uq.dequantize_q8_0, O.dequantize_q8_0)])
def test_dequantize_bit_exact(dtype, fn_uq, fn_or):
    n = 4096 * 64
    w = S.weights(dtype, 64, 4096, seed=dtype)
    got, ref = np.zeros(n, np.float32), np.zeros(n, np.float32)
    fn_uq(got, w)
    fn_or(ref, w)
    assert_bitwise(got, ref, f"dequantize {dtype}")


def test_reference_pin_blocks_dequantize_and_unpack():
    fx = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_pins.json")))
    for name, v in fx["blocks"].items():
        blk = np.array(v["bytes"], np.uint8)
        if blk.size == 144:
            got, ref = np.zeros(256, np.float32), np.zeros(256, np.float32)
            uq.dequantize_q4_k(got, blk)
            O.dequantize_q4_k(ref, blk)
            assert_bitwise(got, ref, name)
        else:
            for g, r in zip(uq.unpack_q6_k(blk), O.unpack_q6_k(blk)):
                assert_bitwise(g, r, name)


def test_quantize_q8_k_bit_exact():
    x = S.activations(256 * 64, seed=3)
    x[0:256] = 0.0                       # zero block
    x[256:512] = 1.0                      # all equal: first index wins
    x[600], x[601] = 5.0, -5.0            # tie, +5 first
    x[800], x[700] = -6.0, 6.0            # tie, +6 first (700 < 800)
    x[1100] = -9.0                        # negative max
    x[2048:2304] *= 1e-20
    got, ref = uq.quantize_q8_k(x), O.quantize_q8_k(x)
    assert_bitwise(got["d"], ref["d"], "q8k d")
    assert np.array_equal(got["qs"], ref["qs"])
    assert np.array_equal(got["bsums"], ref["bsums"])


def _non_finite_x(K, with_inf):
    """N(0,1) activations with a quiet NaN (block 0), a NaN with the sign bit
    set (block 1) and, with_inf, +inf (block 2), -inf (block 3) and a NaN
    beside an infinity (block 4); later blocks are finite."""
    x = S.activations(K, seed=21)
    x[5] = np.float32(np.nan)
    x[256 + 9] = np.uint32(0xFFC00000).view(np.float32)
    if with_inf:
        x[512 + 77] = np.inf
        x[768 + 3] = -np.inf
        x[1024 + 1], x[1024 + 200] = np.nan, np.inf
    return x


def assert_bitwise_or_both_nan(got, ref, what):
    """Bit-exact wherever the reference is a number; NaN exactly where it is
    NaN (the NaN an invalid operation makes is positive on the GPU and
    negative on x86, so NaN bits are not compared)."""
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan), f"{what}: NaN positions differ"
    assert_bitwise(got[~nan], ref[~nan], what)


@pytest.mark.parametrize("with_inf", [False, True])
def test_quantize_q8_k_non_finite_bit_exact(with_inf):
    """quantize_q8_k (quants.rs:250-290) on NaN and infinite activations: the
    strict argmax skips NaN, nearest_int's magic-number add maps a quiet NaN
    product to 0, and a block whose maximum is +-inf gets iscale = -+0 and
    d = -+inf with every quant 0."""
    x = _non_finite_x(4096, with_inf)
    got, ref = uq.quantize_q8_k(x), O.quantize_q8_k(x)
    assert_bitwise(got["d"], ref["d"], "q8k d")
    assert np.array_equal(got["qs"], ref["qs"])
    assert np.array_equal(got["bsums"], ref["bsums"])
    if with_inf:
        assert np.isinf(ref["d"][2]) and np.isinf(ref["d"][3])


@pytest.mark.parametrize("dtype", [S.Q4_K, S.Q6_K])
@pytest.mark.parametrize("with_inf", [False, True])
def test_gemv_quant_q8k_non_finite_activations(dtype, with_inf):
    """gemv_quant_q8k (quants.rs:474-515) with NaN / infinite activations,
    host mirror and batched device launch: NaNs quantize to 0, so such x
    gives the reference's finite outputs bit for bit; an infinity makes the
    block's d infinite and every row NaN, as in the reference."""
    K, N = 4096, 300
    w = S.weights(dtype, N, K, seed=K + N + dtype)
    x = _non_finite_x(K, with_inf)
    ref = np.zeros(N, np.float32)
    O.gemv_quant_q8k(ref, x, w, K, N, dtype)
    assert np.all(np.isnan(ref)) if with_inf else np.all(np.isfinite(ref))
    got = np.zeros(N, np.float32)
    uq.gemv_quant_q8k(got, x, w, K, N, dtype)
    assert_bitwise_or_both_nan(got, ref, f"gemv_quant_q8k dtype {dtype} inf {with_inf}")
    W = uq.Weights(w, dtype, K, N)
    dx, dys = uq.DeviceArray.from_numpy(x), [uq.DeviceArray(4 * N) for _ in range(2)]
    uq.gemv_q8k_batch([W, W], dx, dys)
    for i, dy in enumerate(dys):
        assert_bitwise_or_both_nan(dy.download(np.float32, N), ref, f"q8k batch {i} dtype {dtype} inf {with_inf}")
    W.free()


def test_swiglu_close():
    rng = np.random.default_rng(1)
    g = (rng.standard_normal(1 << 16) * 20).astype(np.float32)
    u = (rng.standard_normal(1 << 16) * 20).astype(np.float32)
    assert_close(uq.swiglu(g, u), O.swiglu(g, u), atol=0, rtol=2e-6, what="swiglu")


# --------------------------------------------------------------- GEMV

GEMV_CASES = [
    (S.Q4_K, 256, 7), (S.Q4_K, 4096, 4096), (S.Q4_K, 4096, 33), (S.Q4_K, 12288, 512),
    (S.Q4_K, 1024, 300),
    # K split over waves, slices streamed through LDS: two and three full
    # slices, a last slice of one or two blocks, uneven rows per group; 16384
    # (four slices) runs the register-fed split
    (S.Q4_K, 8192, 1000), (S.Q4_K, 4352, 77), (S.Q6_K, 4608, 513), (S.Q6_K, 8192, 2000),
    # four and five slices (K up to 20480, beyond the 64 KB layout budget),
    # a last slice of 4 blocks (13312)
    (S.Q4_K, 16384, 64), (S.Q6_K, 16384, 300), (S.Q4_K, 13312, 129), (S.Q4_K, 20480, 200),
    (S.Q6_K, 20480, 97),
    (S.Q6_K, 256, 5), (S.Q6_K, 4096, 4096), (S.Q6_K, 12288, 512), (S.Q6_K, 2048, 301),
    (S.Q8_0, 4096, 4096), (S.Q8_0, 64, 9), (S.Q8_0, 4064, 33),  # K % 64 == 32: generic kernel
    # Q8_0 rows of 256 to 4096 weights (the register-fed kernel)
    (S.Q8_0, 256, 5), (S.Q8_0, 1024, 77), (S.Q8_0, 2048, 301), (S.Q8_0, 3072, 100), (S.Q8_0, 512, 3000),
    (S.F32, 4096, 64),
]


@pytest.mark.parametrize("dtype,K,N", GEMV_CASES)
def test_gemv_quant_parity(dtype, K, N):
    log(f"gemv_quant dtype={dtype} K={K} N={N}")
    w = S.weights(dtype, N, K, seed=K * 31 + N + dtype)
    x = S.activations(K + 5, seed=N + dtype)  # x longer than dim_in (quants.rs:431)
    ref = np.zeros(N, np.float32)
    O.gemv_quant(ref, x, w, K, N, dtype, nthreads=NT)
    got = np.zeros(N, np.float32)
    uq.gemv_quant(got, x, w, K, N, dtype)
    assert_close(got, ref, what=f"gemv dtype {dtype} K {K} N {N}")
    if not _gemv_runs_generic(dtype, K):
        assert_bitwise(got, uq.emu_gemv(x[:K], w, K, N, dtype), "device vs emulation")


def _gemv_runs_generic(dtype, K):
    """True when gemv_quant runs the generic kernel (exact f64 products, not
    the digit-plane path the emulation models): F32 rows, Q8_0 with
    K % 64 != 0, and activation layouts beyond 64 KB of LDS (64-task padded
    planes of 256 bytes per task, Q6_K's 32-byte aux, run scales, group sums)."""
    if dtype == S.F32 or (dtype == S.Q8_0 and K % 64):
        return True
    nt = -(-(K // 64) // 64) * 64  # tasks of 64 activations, rounded to whole waves
    lds = nt * 256 + (nt * 32 if dtype == S.Q6_K else 0) + (K // 128 + 1) * 4 + (K // 32) * 8
    if lds <= 64 * 1024:
        return False
    # the streaming split (Q4_K / Q6_K, 2..5 slices) runs within the CU's 160 KB
    loads = {S.Q4_K: 3, S.Q6_K: 4}.get(dtype, 0)
    ks = -(-(K // 64) // 64)
    if not loads or not 2 <= ks <= 5:
        return True
    ng, d = (4, 2) if ks <= 3 else (3, 1)
    sks = (lds + 15) // 16 * 16 + 2 * ng * ks * 4 * 8 + ks * ng * d * loads * 1024
    return sks > 160 * 1024


@pytest.mark.parametrize("dtype,K,N", [(S.Q4_K, 256, 7), (S.Q4_K, 4096, 4096), (S.Q4_K, 12288, 512),
                                       (S.Q6_K, 256, 5), (S.Q6_K, 4096, 4096), (S.Q6_K, 12288, 512),
                                       (S.Q4_K, 1024, 301), (S.Q6_K, 2048, 33),
                                       (S.Q4_K, 8192, 1000), (S.Q6_K, 12288, 5000), (S.Q6_K, 4352, 77),
                                       (S.Q4_K, 16384, 300), (S.Q6_K, 16384, 77), (S.Q4_K, 13312, 100),
                                       (S.Q6_K, 20480, 50),
                                       (S.Q4_K, 4096, 65636), (S.Q6_K, 3584, 50001), (S.Q6_K, 2048, 50000)])
def test_gemv_quant_q8k_bit_exact(dtype, K, N):
    """Every kernel of the path: rows streamed with one or three tasks per
    lane, the K-split kernel (two to five slices; a last slice of one or four
    blocks; row groups with uneven or no rows in the last workgroups), and
    long launches (16 or more rows per wave, the rotating wave priority)
    beside the full head."""
    log(f"gemv_quant_q8k dtype={dtype} K={K} N={N}")
    w = S.weights(dtype, N, K, seed=K * 17 + N + dtype)
    x = S.activations(K, seed=N * 3 + dtype)
    ref = np.zeros(N, np.float32)
    O.gemv_quant_q8k(ref, x, w, K, N, dtype, nthreads=NT)
    got = np.zeros(N, np.float32)
    uq.gemv_quant_q8k(got, x, w, K, N, dtype)
    assert_bitwise(got, ref, f"q8k dtype {dtype} K {K}")


@pytest.mark.parametrize("dtype,K,N", [(S.Q4_K, 4096, 64), (S.Q6_K, 4096, 64), (S.Q6_K, 12288, 64),
                                       (S.Q4_K, 12288, 64)])
def test_gemv_quant_q8k_special_block_scales(dtype, K, N):
    """Blocks whose f16 d (and Q4_K dmin) is subnormal, the largest finite,
    zero, negative, infinite or NaN: the epilogue's f16 decode matches the
    reference's f16_to_f32 (quants.rs:44-72). Finite outputs are compared
    bit for bit; the rows a NaN or infinite scale reaches are NaN in both."""
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
        if dtype == S.Q4_K and r % 3 == 0:  # dmin too
            v2 = specials[(r // 3) % len(specials)]
            w[r, blk * bb + 2] = v2 & 0xFF
            w[r, blk * bb + 3] = v2 >> 8
    w = w.reshape(-1)
    x = S.activations(K, seed=N + 5)
    ref = np.zeros(N, np.float32)
    O.gemv_quant_q8k(ref, x, w, K, N, dtype, nthreads=NT)
    got = np.zeros(N, np.float32)
    uq.gemv_quant_q8k(got, x, w, K, N, dtype)
    nan_r, nan_g = np.isnan(ref), np.isnan(got)
    assert np.array_equal(nan_r, nan_g), f"NaN rows differ: ref {np.nonzero(nan_r)[0][:8]} got {np.nonzero(nan_g)[0][:8]}"
    assert nan_r.any(), "the test plants infinite and NaN scales"
    assert_bitwise(got[~nan_r], ref[~nan_r], f"q8k special scales dtype {dtype} K {K}")


def _edge_activations(K):
    """The edge-case vector of test_cpu_emulation (zero run, tiny run, one
    huge outlier, subnormals, a sign-flipped scaled block), tiled over K."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(K).astype(np.float32)
    for base in range(0, K, 4096):
        x[base:base + 32] = 0.0
        x[base + 64:base + 96] *= 1e-30
        x[base + 96] = 3e4
        x[base + 200:base + 232] = np.float32(1e-41)  # subnormal f32
        x[base + 512:base + 1024] *= -1e3
    return x


@pytest.mark.parametrize("dtype,K,N", [(S.Q4_K, 4096, 17), (S.Q6_K, 4096, 17), (S.Q8_0, 4096, 17),
                                       (S.Q4_K, 4096, 4096), (S.Q6_K, 4096, 3000), (S.Q4_K, 12288, 700),
                                       (S.Q6_K, 12288, 700), (S.Q8_0, 12288, 300), (S.Q4_K, 16384, 200)])
def test_gemv_activation_edge_cases_on_device(dtype, K, N):
    """The fixed-point activation form on the device with outliers, zero and
    tiny runs and subnormals: within the gemv_quant tolerance of the oracle,
    and equal to the CPU emulation of the same kernel code bit for bit."""
    log(f"gemv edge activations dtype={dtype} K={K} N={N}")
    w = S.weights(dtype, N, K, seed=77 + K + N)
    x = _edge_activations(K)
    ref = np.zeros(N, np.float32)
    O.gemv_quant(ref, x, w, K, N, dtype, nthreads=NT)
    got = np.zeros(N, np.float32)
    uq.gemv_quant(got, x, w, K, N, dtype)
    assert_close(got, ref, what=f"edge activations dtype {dtype} K {K}")
    if not _gemv_runs_generic(dtype, K):
        assert_bitwise(got, uq.emu_gemv(x, w, K, N, dtype), "device vs emulation")


@pytest.mark.parametrize("dtype,K,N", [(S.Q4_K, 4096, 300), (S.Q6_K, 4096, 300), (S.Q8_0, 4096, 300),
                                       (S.Q4_K, 12288, 300), (S.Q6_K, 12288, 300)])
@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_gemv_non_finite_activation_gives_nan_on_device(dtype, K, N, bad):
    """A NaN or infinite activation: every output row is NaN (gemv_quant's
    rows are NaN, or +-inf / NaN for an infinity), never a finite number;
    the batched launch and the device-handle path agree."""
    w = S.weights(dtype, N, K, seed=K + N)
    x = S.activations(K, seed=3)
    x[K // 3] = bad
    got = np.zeros(N, np.float32)
    uq.gemv_quant(got, x, w, K, N, dtype)
    assert np.all(np.isnan(got))
    W = uq.Weights(w, dtype, K, N)
    dx, dy = uq.DeviceArray.from_numpy(x), uq.DeviceArray(4 * N)
    uq.gemv_batch([W], dx, [dy])
    assert np.all(np.isnan(dy.download(np.float32, N)))


def test_reference_pins_through_gemv():
    fx = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_pins.json")))
    i = np.arange(256)
    xp = ((i * 7919) % 1009).astype(np.float32) / np.float32(1009.0) - np.float32(0.5)
    xa = ((i * 31 + 17) % 257).astype(np.float32) / np.float32(257.0) - np.float32(0.5)
    for case in fx["cases"]:
        blk = np.array(fx["blocks"][case["block"]]["bytes"], np.uint8)
        dt = uq.DType.Q6K if blk.size == 210 else uq.DType.Q4K
        for x, key in ((xp, "dot_x_pattern"), (xa, "dot_x_alt")):
            y = np.zeros(1, np.float32)
            uq.gemv_quant(y, x, blk, 256, 1, dt)
            assert abs(float(y[0]) - case[key]) < fx["tolerance"], (case["block"], key)
            y8 = np.zeros(1, np.float32)
            uq.gemv_quant_q8k(y8, x, blk, 256, 1, dt)
            r8 = np.zeros(1, np.float32)
            O.gemv_quant_q8k(r8, x, blk, 256, 1, dt)
            assert_bitwise(y8, r8, case["block"])


# --------------------------------------------------------------- device API

def test_device_api_gemv_and_q8k_full_head():
    """Config: Q6_K output projection 152064 x 4096, weights device-resident."""
    K, N = 4096, 152064
    log("head: generating 511 MB of Q6_K blocks")
    w = S.weights(S.Q6_K, N, K, seed=S.seed_for(1))
    x = S.activations(K, seed=S.seed_for(1))
    W = uq.Weights(w, uq.DType.Q6K, K, N)
    dx, dy = uq.DeviceArray.from_numpy(x), uq.DeviceArray(4 * N)
    uq.gemv(W, dx, dy)
    got = dy.download(np.float32, N)
    log("head: oracle")
    ref = np.zeros(N, np.float32)
    O.gemv_quant(ref, x, w, K, N, S.Q6_K, nthreads=NT)
    assert_close(got, ref, what="head gemv")
    uq.gemv_q8k(W, dx, dy)
    got8 = dy.download(np.float32, N)
    ref8 = np.zeros(N, np.float32)
    O.gemv_quant_q8k(ref8, x, w, K, N, S.Q6_K, nthreads=NT)
    assert_bitwise(got8, ref8, "head q8k")
    W.free()


def test_device_api_ffn_swiglu():
    """Config: gate/up Q4_K 12288 x 4096 with SwiGLU in the epilogue, down
    Q6_K 4096 x 12288 (qwen35_forward.rs:713-768).
    The GEMV outputs g = gate.x, u = up.x meet the gemv_quant tolerance; the
    fused epilogue equals swiglu (kernels.rs:174-182, device expf) of those
    same GEMV outputs bit for bit; h stays within the reference's tolerance
    propagated through swiglu (d silu/dg and silu(g) amplify the allowed
    GEMV error); down meets the tolerance on the device's own h."""
    n, nff = 4096, 12288
    g = S.weights(S.Q4_K, nff, n, seed=S.seed_for(2, 1))
    u = S.weights(S.Q4_K, nff, n, seed=S.seed_for(2, 2))
    d = S.weights(S.Q6_K, n, nff, seed=S.seed_for(2, 3))
    x = S.activations(n, seed=S.seed_for(2))
    G, U, D = uq.Weights(g, uq.DType.Q4K, n, nff), uq.Weights(u, uq.DType.Q4K, n, nff), uq.Weights(d, uq.DType.Q6K, nff, n)
    dx, dh, dy = uq.DeviceArray.from_numpy(x), uq.DeviceArray(4 * nff), uq.DeviceArray(4 * n)
    uq.ffn_swiglu(G, U, D, dx, dh, dy)
    h, y = dh.download(np.float32, nff), dy.download(np.float32, n)
    dg, du = uq.DeviceArray(4 * nff), uq.DeviceArray(4 * nff)
    uq.gemv(G, dx, dg)
    uq.gemv(U, dx, du)
    gd, ud = dg.download(np.float32, nff), du.download(np.float32, nff)
    rg, ru = np.zeros(nff, np.float32), np.zeros(nff, np.float32)
    O.gemv_quant(rg, x, g, n, nff, S.Q4_K, nthreads=NT)
    O.gemv_quant(ru, x, u, n, nff, S.Q4_K, nthreads=NT)
    assert_close(gd, rg, what="ffn gate")
    assert_close(ud, ru, what="ffn up")
    assert_bitwise(h, uq.swiglu(gd, ud), "fused epilogue vs swiglu of the GEMV outputs")
    rh = O.swiglu(rg, ru).astype(np.float64)
    g64, u64 = rg.astype(np.float64), ru.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-g64))
    dsilu = sig * (1.0 + g64 * (1.0 - sig))
    tol_g, tol_u = 1e-4 + 1e-3 * np.abs(g64), 1e-4 + 1e-3 * np.abs(u64)
    bound = 1e-4 + 1e-3 * np.abs(rh) + np.abs(dsilu * u64) * tol_g + np.abs(g64 * sig) * tol_u
    assert np.all(np.abs(h - rh) <= bound), "h outside the propagated tolerance"
    ry = np.zeros(n, np.float32)
    O.gemv_quant(ry, h, d, nff, n, S.Q6_K, nthreads=NT)
    assert_close(y, ry, what="ffn down")


def test_device_api_q8_0_projection():
    K, N = 4096, 4096
    w = S.weights(S.Q8_0, N, K, seed=S.seed_for(2, 4))
    x = S.activations(K, seed=S.seed_for(2, 5))
    W = uq.Weights(w, uq.DType.Q8_0, K, N)
    dx, dy = uq.DeviceArray.from_numpy(x), uq.DeviceArray(4 * N)
    uq.gemv(W, dx, dy)
    ref = np.zeros(N, np.float32)
    O.gemv_quant(ref, x, w, K, N, S.Q8_0, nthreads=NT)
    assert_close(dy.download(np.float32, N), ref, what="q8_0 projection")


def test_device_dequantize_handle():
    K, N = 4096, 256
    w = S.weights(S.Q4_K, N, K, seed=5)
    W = uq.Weights(w, uq.DType.Q4K, K, N)
    d = uq.DeviceArray(4 * K * N)
    uq.dequantize(W, d)
    uq.synchronize()
    ref = np.zeros(K * N, np.float32)
    O.dequantize_q4_k(ref, w)
    assert_bitwise(d.download(np.float32, K * N), ref, "device dequantize")


# ------------------------------------------------- embedding GET_ROWS (f4)

def _embed_ref(dtype, w, K, tokens):
    """embed (min_forward.rs:160-184) restated with the oracle: each token's
    row dequantized by itself (F32 rows copied)."""
    rb = uq.row_bytes(dtype, K)
    out = np.zeros((len(tokens), K), np.float32)
    for r, t in enumerate(tokens):
        row = w[t * rb:(t + 1) * rb]
        if dtype == S.F32:
            out[r] = row.view(np.float32)
        else:
            out[r] = O.dequantize(dtype, row, K)
    return out


@pytest.mark.parametrize("dtype,K,V,n", [(S.Q4_K, 4096, 1000, 300), (S.Q4_K, 256, 3, 7), (S.F32, 1000, 50, 9),
                                         (S.Q6_K, 4096, 64, 20), (S.Q8_0, 2048, 64, 20)])
def test_embed_rows_bit_exact(dtype, K, V, n):
    rng = np.random.default_rng(K + V + n)
    if dtype == S.F32:
        w = rng.standard_normal(V * K).astype(np.float32).view(np.uint8)
    else:
        w = S.weights(dtype, V, K, seed=V)
    # first, last, repeated ids and a run that crosses the 256-id launch chunk
    tokens = np.concatenate([[0, V - 1, 1 % V, 1 % V], rng.integers(0, V, max(0, n - 4))]).astype(np.uint32)[:n]
    W = uq.Weights(w, dtype, K, V)
    d = uq.DeviceArray(4 * n * K)
    uq.embed(W, tokens, d)
    uq.synchronize()
    got = d.download(np.float32, n * K).reshape(n, K)
    assert_bitwise(got, _embed_ref(dtype, w, K, tokens), f"embed dtype={dtype} K={K} n={n}")


def test_embed_refuses_out_of_vocab_before_writing():
    K, V = 256, 10
    w = S.weights(S.Q4_K, V, K, seed=2)
    W = uq.Weights(w, S.Q4_K, K, V)
    d = uq.DeviceArray(4 * 3 * K)
    sentinel = np.full(3 * K, 7.0, np.float32)
    d.upload(sentinel)
    with pytest.raises(uq.UqError) as e:
        uq.embed(W, [1, V, 2], d)
    assert e.value.kind == "TOKEN" and "10" in str(e.value)
    uq.embed(W, [], d)  # no tokens: no-op
    uq.synchronize()
    assert_bitwise(d.download(np.float32, 3 * K), sentinel, "untouched after refusal")


# --------------------------------------------------- GGUF -> HBM loader (f2)

def test_gguf_file_to_hbm_gemv_and_embed(tmp_path):
    """A GGUF file written byte by byte, mapped by uq_gguf_open, its tensors
    uploaded unchanged: the GEMVs and the embedding lookup on the uploaded
    handles equal the oracle on the file's bytes."""
    from uq import gguf as G
    K, V, N = 4096, 512, 1024
    emb = S.weights(S.Q4_K, V, K, seed=41)
    head = S.weights(S.Q6_K, V, K, seed=42)
    up = S.weights(S.Q4_K, N, K, seed=43)
    path = tmp_path / "tiny.gguf"
    path.write_bytes(G.write([("general.architecture", G.STRING, "qwen35")],
                             [("token_embd.weight", [K, V], S.Q4_K, emb), ("output.weight", [K, V], S.Q6_K, head),
                              ("blk.0.ffn_up.weight", [K, N], S.Q4_K, up)]))
    with G.Gguf.open(path) as g:
        assert g.check("blk.0.ffn_up.weight", K * N, [uq.DType.Q4K]) == uq.DType.Q4K
        Wh, Wu, We = g.upload("output.weight"), g.upload("blk.0.ffn_up.weight"), g.upload("token_embd.weight")
    assert (Wh.dtype, Wh.dim_in, Wh.dim_out) == (S.Q6_K, K, V) and (Wu.dim_in, Wu.dim_out) == (K, N)
    x = S.activations(K, seed=44)
    dx = uq.DeviceArray.from_numpy(x)
    for W, w, n in ((Wh, head, V), (Wu, up, N)):
        dy = uq.DeviceArray(4 * n)
        uq.gemv_q8k(W, dx, dy)
        uq.synchronize()
        ref = np.zeros(n, np.float32)
        O.gemv_quant_q8k(ref, x, w, K, n, W.dtype, nthreads=NT)
        assert_bitwise(dy.download(np.float32, n), ref, f"gguf-loaded gemv_q8k dtype={W.dtype}")
    toks = np.array([3, V - 1, 0, 3], np.uint32)
    de = uq.DeviceArray(4 * len(toks) * K)
    uq.embed(We, toks, de)
    uq.synchronize()
    assert_bitwise(de.download(np.float32, len(toks) * K).reshape(len(toks), K),
                   _embed_ref(S.Q4_K, emb, K, toks), "gguf-loaded embed")


def test_device_api_errors():
    w = S.weights(S.Q8_0, 4, 64, seed=1)
    W = uq.Weights(w, uq.DType.Q8_0, 64, 4)
    dx, dy = uq.DeviceArray(256), uq.DeviceArray(16)
    with pytest.raises(uq.UqError) as e:
        uq.gemv_q8k(W, dx, dy)
    assert e.value.kind == "DTYPE"
    with pytest.raises(uq.UqError) as e:
        uq.Weights(w[:-1], uq.DType.Q8_0, 64, 4)
    assert e.value.kind == "LEN"


@pytest.mark.parametrize("dtype,K,ns", [(S.Q4_K, 4096, (8192, 4096, 32, 32)), (S.Q6_K, 4096, (8192, 1024, 1024)),
                                        (S.Q4_K, 12288, (4096, 7)), (S.Q8_0, 4096, (100, 4096)),
                                        (S.Q6_K, 16384, (1000, 33))])
def test_gemv_batch_equals_separate_gemvs(dtype, K, ns):
    """uq_gemv_batch: one launch over several weight tensors sharing x writes
    exactly what separate uq_gemv calls write (same per-row arithmetic), and
    each is within the gemv_quant tolerance of the oracle."""
    x = S.activations(K, seed=K + len(ns))
    dx = uq.DeviceArray.from_numpy(x)
    ws = [S.weights(dtype, n, K, seed=17 * i + n) for i, n in enumerate(ns)]
    Ws = [uq.Weights(w, dtype, K, n) for w, n in zip(ws, ns)]
    yb = [uq.DeviceArray(4 * n) for n in ns]
    ys = [uq.DeviceArray(4 * n) for n in ns]
    uq.gemv_batch(Ws, dx, yb)
    for W, y in zip(Ws, ys):
        uq.gemv(W, dx, y)
    for w, n, a, b in zip(ws, ns, yb, ys):
        got, sep = a.download(np.float32, n), b.download(np.float32, n)
        assert_bitwise(got, sep, what=f"batch vs separate n={n}")
        ref = np.zeros(n, np.float32)
        O.gemv_quant(ref, x, w, K, n, dtype, nthreads=NT)
        assert_close(got, ref, what=f"batch n={n}")


def test_gemv_batch_rejects_mixed_shapes():
    K = 4096
    a = uq.Weights(S.weights(S.Q4_K, 8, K, seed=1), uq.DType.Q4K, K, 8)
    b = uq.Weights(S.weights(S.Q6_K, 8, K, seed=2), uq.DType.Q6K, K, 8)
    c = uq.Weights(S.weights(S.Q4_K, 8, 2 * K, seed=3), uq.DType.Q4K, 2 * K, 8)
    dx = uq.DeviceArray.from_numpy(S.activations(2 * K, seed=4))
    ys = [uq.DeviceArray(32), uq.DeviceArray(32)]
    for pair in ((a, b), (a, c)):
        with pytest.raises(uq.UqError) as e:
            uq.gemv_batch(list(pair), dx, ys)
        assert e.value.kind == "LEN"


@pytest.mark.parametrize("dtype,K,ns", [(S.Q4_K, 4096, (12288, 12288)), (S.Q6_K, 4096, (8192, 1024, 1024)),
                                        (S.Q4_K, 12288, (4096, 33))])
def test_gemv_q8k_batch_bit_exact(dtype, K, ns):
    """uq_gemv_q8k_batch: every output equals gemv_quant_q8k bit for bit (and
    the separate uq_gemv_q8k launches)."""
    x = S.activations(K, seed=K + 3 * len(ns))
    dx = uq.DeviceArray.from_numpy(x)
    ws = [S.weights(dtype, n, K, seed=31 * i + n) for i, n in enumerate(ns)]
    Ws = [uq.Weights(w, dtype, K, n) for w, n in zip(ws, ns)]
    yb = [uq.DeviceArray(4 * n) for n in ns]
    uq.gemv_q8k_batch(Ws, dx, yb)
    for w, W, n, a in zip(ws, Ws, ns, yb):
        ref = np.zeros(n, np.float32)
        O.gemv_quant_q8k(ref, x, w, K, n, dtype, nthreads=NT)
        assert_bitwise(a.download(np.float32, n), ref, what=f"q8k batch n={n}")
        ys = uq.DeviceArray(4 * n)
        uq.gemv_q8k(W, dx, ys)
        assert_bitwise(ys.download(np.float32, n), ref, what=f"q8k separate n={n}")


@pytest.mark.parametrize("down_dtype", [S.Q4_K, S.Q6_K])
def test_ffn_swiglu_q8k_is_the_reference_ffn_bit_for_bit(down_dtype):
    """uq_ffn_swiglu_q8k reproduces Qwen35Forward::ffn (qwen35_forward.rs:735-765):
    g, u = gemv_quant_q8k(gate/up, p), sw = swiglu(g, u), f = gemv_quant_q8k(down, sw),
    every intermediate bit for bit."""
    n, nff = 4096, 12288
    gw = S.weights(S.Q4_K, nff, n, seed=41)
    uw = S.weights(S.Q4_K, nff, n, seed=42)
    dw = S.weights(down_dtype, n, nff, seed=43)
    x = S.activations(n, seed=44)
    G, U, D = (uq.Weights(gw, uq.DType.Q4K, n, nff), uq.Weights(uw, uq.DType.Q4K, n, nff),
               uq.Weights(dw, down_dtype, nff, n))
    dx = uq.DeviceArray.from_numpy(x)
    dg, du, dh, dy = uq.DeviceArray(4 * nff), uq.DeviceArray(4 * nff), uq.DeviceArray(4 * nff), uq.DeviceArray(4 * n)
    uq.ffn_swiglu_q8k(G, U, D, dx, dg, du, dh, dy)
    g = np.zeros(nff, np.float32)
    u = np.zeros(nff, np.float32)
    O.gemv_quant_q8k(g, x, gw, n, nff, S.Q4_K, nthreads=NT)
    O.gemv_quant_q8k(u, x, uw, n, nff, S.Q4_K, nthreads=NT)
    sw = O.swiglu(g, u)
    assert_bitwise(dg.download(np.float32, nff), g, what="ffn g")
    assert_bitwise(du.download(np.float32, nff), u, what="ffn u")
    # swiglu's expf is the platform libm's in the reference (f32::exp); the
    # device expf and the oracle's glibc expf agree within 1-2 ulp, so h is
    # checked to 2 ulp and the down projection bit for bit on the device's h
    h = dh.download(np.float32, nff)
    ulp = np.abs(h.view(np.int32).astype(np.int64) - sw.view(np.int32).astype(np.int64))
    assert int(ulp.max()) <= 2, f"swiglu ulp {int(ulp.max())}"
    f = np.zeros(n, np.float32)
    O.gemv_quant_q8k(f, h, dw, nff, n, down_dtype, nthreads=NT)
    assert_bitwise(dy.download(np.float32, n), f, what="ffn out")


def test_swiglu_device_arrays_match_uq_swiglu_and_oracle():
    """uq_swiglu_d equals the host-pointer uq_swiglu bit for bit, and the
    oracle (glibc expf) within 2 ulp over a wide range of gate values."""
    n = 12345
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(n) * 30).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    dg, du, dh = uq.DeviceArray.from_numpy(g), uq.DeviceArray.from_numpy(u), uq.DeviceArray(4 * n)
    uq.swiglu_d(dh, dg, du, n)
    h = dh.download(np.float32, n)
    assert_bitwise(h, uq.swiglu(g, u), what="swiglu_d vs uq_swiglu")
    ref = O.swiglu(g, u)
    ulp = np.abs(h.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert int(ulp.max()) <= 2, f"swiglu ulp {int(ulp.max())}"
