"""Pins the CPU oracle before the GPU results are compared with it.

Three kinds of evidence, per function:
  * the reference's own known-answer tests, restated with their values
    (crates/unltd-tensor/src/quants.rs:582-1222, kernels.rs:434-447,
    :595-611, min_forward.rs:270-303);
  * the reference's real-byte pins: four GGUF blocks whose dots were computed
    by gguf-py's independent dequantizer (fixture tests/golden/reference_pins.json);
  * checks the mathematics fixes independently of the oracle's code: numpy's
    own f16 decoder, GGUF block ENCODERS (the packing direction, written
    from the format, not from the decoder), exact integer arithmetic on
    inputs where every float operation is exact, and np.rint as an
    independent round-half-even.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
F16_ONE, F16_TWO = 0x3C00, 0x4000


def q4_block(d, dmin, scales, qs):
    """quants.rs:686-694: d, dmin (f16 bits), scales[12], qs[128]."""
    b = bytearray()
    b += int(d).to_bytes(2, "little") + int(dmin).to_bytes(2, "little")
    b += bytes(scales) + bytes(qs)
    assert len(b) == 144
    return bytes(b)


def q6_block(d, ql, qh, scales):
    """quants.rs:696-705: ql[128], qh[64], scales[16] (i8), d LAST."""
    b = bytearray(bytes(ql) + bytes(qh) + bytes(np.array(scales, np.int8).view(np.uint8)))
    b += int(d).to_bytes(2, "little")
    assert len(b) == 210
    return bytes(b)


# ---------------------------------------------------------------- a1: f16

def test_f16_to_f32_known_patterns():  # quants.rs:582-596
    f = O.f16_to_f32
    assert f(0x3C00) == 1.0 and f(0x4000) == 2.0 and f(0xC000) == -2.0
    assert f(0x0000) == 0.0
    assert np.float32(f(0x8000)).view(np.uint32) == 0x80000000
    assert math.isinf(f(0x7C00)) and f(0x7C00) > 0
    assert math.isinf(f(0xFC00)) and f(0xFC00) < 0
    assert math.isnan(f(0x7E00))
    assert f(0x0001) == 2.0 ** -24
    assert f(0x03FF) == 2.0 ** -14 - 2.0 ** -24
    assert f(0x7BFF) == 65504.0
    assert f(0x3555) == 0.333251953125


def test_f16_to_f32_exhaustive_vs_numpy():
    """All 65536 patterns against numpy's independent half decoder. The only
    allowed difference is the NaN payload, which the reference canonicalises
    to a quiet NaN with zero payload (quants.rs:66)."""
    h = np.arange(65536, dtype=np.uint32)
    import ctypes
    L = O.lib()
    got = np.array([L.or_f16_to_f32(int(v)) for v in h], dtype=np.float32).view(np.uint32)
    ref = h.astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    nan = ((h >> 10) & 0x1F == 0x1F) & (h & 0x3FF != 0)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all(got[nan] == ((h[nan] >> 15) << 31 | 0x7FC00000))


# ---------------------------------------------------------------- a2: scales

def pack_q4k_scales(sc, m):
    """GGUF Q4_K scale packing, written in the ENCODE direction: 6-bit sc/m of
    groups 0..3 in the low 6 bits of bytes 0..3 / 4..7; groups 4..7 keep their
    low nibbles in bytes 8..11 (sc low, m high) and their top 2 bits in the
    top 2 bits of bytes 0..3 (sc) and 4..7 (m)."""
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] |= sc[j]
            s[j + 4] |= m[j]
        else:
            s[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    return bytes(s)


def test_scale_min_k4_roundtrip_against_encoder():
    rng = np.random.default_rng(1)
    for _ in range(2000):
        sc = rng.integers(0, 64, 8).tolist()
        m = rng.integers(0, 64, 8).tolist()
        s = pack_q4k_scales(sc, m)
        for g in range(8):
            assert O.scale_min_k4(s, g) == (sc[g], m[g])


def test_scale_min_k4_hand_group4():  # quants.rs:730-742 (sc=49, m=19)
    s = bytearray(12)
    s[0], s[4], s[8] = 0xC0, 0x43, 0x31
    assert O.scale_min_k4(bytes(s), 4) == (49, 19)


# ---------------------------------------------------------------- a6: pairwise tree

def test_pairwise_partition_is_the_documented_tree():  # kernels.rs:434-447
    assert O.pairwise_sum_f64([1.0, 2.0, 3.0, 4.0, 5.0]) == 15.0
    assert O.pairwise_sum_f64([1e16, 1.0, -1e16, 1.0]) == 0.0  # serial would give 1
    assert O.pairwise_sum_f64([1.0, 2.0, 3.0]) == 6.0
    assert O.pairwise_sum_f64([]) == 0.0


def test_pairwise_odd_tail_carried_up():
    # n=5 tree is ((a0+a1)+(a2+a3))+a4: the carried tail a4 = -H meets the
    # whole left subtree, where H has already absorbed the small terms -> 0.
    # A tree pairing the tail early, (a0+a1)+((a2+a3)+a4), gives 2.
    H = 2.0 ** 60
    v = [1.0, 1.0, 1.0, H, -H]
    assert O.pairwise_sum_f64(v) == 0.0
    assert (1.0 + 1.0) + ((1.0 + H) + -H) == 2.0
    # n=3: (a0+a1)+a2, not a0+(a1+a2)
    assert O.pairwise_sum_f64([H, -H, 1.0]) == 1.0


def test_dot_f32_small_exact():  # quants.rs:598-604
    assert O.dot_f32([1, 2, 3, 4], [5, 6, 7, 8]) == 70.0
    assert O.dot_f32([1, 2, 3], [4, 5, 6]) == 32.0


# ---------------------------------------------------------------- a3/a7/a14: Q4_K

def test_dequantize_q4_k_hand_values_and_multi_block():  # quants.rs:606-648
    scales = bytearray(12)
    scales[0], scales[4], scales[1], scales[5] = 1, 3, 2, 1
    qs = bytearray(128)
    qs[0] = 0x12
    a = q4_block(F16_ONE, F16_TWO, scales, qs)
    b = q4_block(0, 0, bytes(12), bytes([0xAB] * 128))
    out = np.zeros(512, np.float32)
    O.dequantize_q4_k(out, a + b)
    assert out[0] == -4.0 and out[1] == -6.0 and out[31] == -6.0
    assert out[32] == 0.0 and out[33] == -2.0
    assert np.all(out[64:512] == 0.0)
    x = np.full(256, 0.5, np.float32)
    assert abs(O.dot_f32(x, out[:256]) - O.dot_q4_k(x, a)) < 1e-4


def test_dequantize_q4_k_matches_reference_formula_bitwise():  # quants.rs:650-684
    scales = [0x1F, 0x2E, 0x3D, 0x4C, 0x5B, 0x6A, 0x79, 0x03, 0x92, 0x81, 0x70, 0x6F]
    qs = [(i * 7 + 3) & 0xFF for i in range(128)]
    blk = q4_block(0x3B21, 0x2C10, scales, qs)
    out = np.zeros(256, np.float32)
    O.dequantize_q4_k(out, blk)
    d, mn = O.f16_to_f32(0x3B21), O.f16_to_f32(0x2C10)
    e = 0
    for isx in range(0, 8, 2):
        pair = qs[32 * (isx // 2): 32 * (isx // 2) + 32]
        for g, shift in ((isx, 0), (isx + 1, 4)):
            sc, m = O.scale_min_k4(bytes(scales), g)
            dg, mg = np.float32(d) * np.float32(sc), np.float32(mn) * np.float32(m)
            for l in range(32):
                exp = np.float32(dg * np.float32((pair[l] >> shift) & 0xF)) - mg
                assert np.float32(out[e]).view(np.uint32) == np.float32(exp).view(np.uint32), e
                e += 1


def test_q4_k_zero_block_and_hand_values():  # quants.rs:707-743
    x = np.full(256, 0.5, np.float32)
    assert O.dot_q4_k(x, q4_block(F16_ONE, 0, bytes(12), bytes([0xFF] * 128))) == 0.0
    scales = bytearray(12)
    scales[0], scales[4] = 1, 3
    qs = bytearray(128)
    qs[0] = 0x01
    blk = q4_block(F16_ONE, F16_TWO, scales, qs)
    x = np.zeros(256, np.float32)
    x[0] = 1.0
    assert O.dot_q4_k(x, blk) == -5.0
    x[0], x[1] = 0.0, 1.0
    assert O.dot_q4_k(x, blk) == -6.0
    scales = bytearray(12)
    scales[0], scales[4], scales[8] = 0xC0, 0x43, 0x31
    qs = bytearray(128)
    qs[64] = 0x01
    blk = q4_block(F16_ONE, F16_ONE, scales, qs)
    x = np.zeros(256, np.float32)
    x[128] = 1.0
    assert O.dot_q4_k(x, blk) == 30.0


def test_q4_k_pairwise_tree_is_the_contract():  # quants.rs:745-766
    scales = bytearray(12)
    scales[0] = 1
    qs = bytearray(128)
    qs[0:4] = bytes([0x0A, 0x01, 0x0A, 0x01])
    blk = q4_block(F16_ONE, 0, scales, qs)
    x = np.zeros(256, np.float32)
    x[0:4] = [1e19, 1.0, -1e19, 1.0]
    assert O.dot_q4_k(x, blk) == 0.0


def test_q4_k_full_block_matches_layout_reference():  # quants.rs:768-788
    qs = bytes(range(128))
    blk = q4_block(F16_ONE, 0, bytes([1] * 12), qs)
    x = np.arange(1, 257, dtype=np.float32)
    exp = 0.0
    for e in range(256):
        g = e // 32
        byte = qs[32 * (g // 2) + e % 32]
        exp += (e + 1) * ((byte & 0xF) if g % 2 == 0 else (byte >> 4))
    assert O.dot_q4_k(x, blk) == exp


def test_q4_k_multiblock_stride():  # quants.rs:790-802
    qs = bytearray(128)
    qs[0] = 1
    w = q4_block(F16_ONE, 0, bytes([1] * 12), qs) + q4_block(F16_TWO, 0, bytes([1] * 12), qs)
    assert O.dot_q4_k(np.ones(512, np.float32), w) == 3.0


# ---------------------------------------------------------------- a4/a8: Q6_K

def test_q6_k_zero_block_and_hand_values():  # quants.rs:804-872
    x = np.full(256, 0.5, np.float32)
    assert O.dot_q6_k(x, q6_block(F16_TWO, [0xFF] * 128, [0xFF] * 64, [0] * 16)) == 0.0

    def one_hot(i):
        v = np.zeros(256, np.float32)
        v[i] = 1.0
        return v

    ql = [0] * 128
    ql[0] = 0x01
    assert O.dot_q6_k(one_hot(0), q6_block(F16_TWO, ql, [0] * 64, [1] * 16)) == -62.0
    ql, qh, sc = [0] * 128, [0] * 64, [0] * 16
    ql[32], qh[0], sc[2] = 0x03, 0x04, -1
    assert O.dot_q6_k(one_hot(32), q6_block(F16_TWO, ql, qh, sc)) == 26.0
    ql, qh, sc = [0] * 128, [0] * 64, [0] * 16
    ql[0], qh[0], sc[4] = 0x50, 0x10, 3
    assert O.dot_q6_k(one_hot(64), q6_block(F16_TWO, ql, qh, sc)) == -66.0
    ql, qh, sc = [0] * 128, [0] * 64, [1] * 16
    ql[32], qh[0] = 0x70, 0x40
    assert O.dot_q6_k(one_hot(96), q6_block(F16_TWO, ql, qh, sc)) == -18.0
    ql, qh, sc = [0] * 128, [0] * 64, [0] * 16
    ql[64], qh[32], sc[8] = 0x02, 0x02, 5
    assert O.dot_q6_k(one_hot(128), q6_block(F16_TWO, ql, qh, sc)) == 20.0


def test_q6_k_pairwise_tree_is_the_contract():  # quants.rs:874-901
    ql = [0] * 128
    ql[0:4] = [0x0A, 0x01, 0x0A, 0x01]
    qh = [0] * 64
    qh[0:4] = [0x02] * 4
    sc = [0] * 16
    sc[0] = 1
    x = np.zeros(256, np.float32)
    x[0:4] = [1e19, 1.0, -1e19, 1.0]
    assert O.dot_q6_k(x, q6_block(F16_ONE, ql, qh, sc)) == 0.0


def test_q6_k_full_block_matches_layout_reference():  # quants.rs:903-934
    ql, qh = list(range(128)), list(range(64))
    sc = [i - 8 for i in range(16)]
    x = np.arange(1, 257, dtype=np.float32)
    exp = 0.0
    for e in range(256):
        byte = ql[64 * (e // 128) + e % 64]
        nib = (byte & 0xF) if (e // 64) % 2 == 0 else (byte >> 4)
        hi2 = (qh[e % 32 + 32 * (e // 128)] >> (2 * ((e % 128) // 32))) & 3
        exp += (e + 1) * sc[e // 16] * ((nib | (hi2 << 4)) - 32)
    assert O.dot_q6_k(x, q6_block(F16_ONE, ql, qh, sc)) == exp


def test_q6_k_multiblock_stride():  # quants.rs:936-952
    ql = [0] * 128
    ql[0] = 1
    sc = [0] * 16
    sc[0] = 1
    w = q6_block(F16_ONE, ql, [0] * 64, sc) + q6_block(F16_TWO, ql, [0] * 64, sc)
    assert O.dot_q6_k(np.ones(512, np.float32), w) == -511.0 + -1022.0


# ------------------------------------------- encoders: independent layout pins

def encode_q4_k(d16, dmin16, sc, m, q):
    """GGUF Q4_K packing in the ENCODE direction: for each 64-element chunk j,
    byte l (l<32) holds element j+l in the low nibble and j+32+l high."""
    qs = bytearray(128)
    for j in range(0, 256, 64):
        for l in range(32):
            qs[j // 2 + l] = q[j + l] | (q[j + 32 + l] << 4)
    return q4_block(d16, dmin16, pack_q4k_scales(sc, m), qs)


def encode_q6_k(d16, sc, L):
    """GGUF Q6_K packing in the ENCODE direction (L = raw 6-bit 0..63): per
    128-element half, ql[l] = L[l] | L[l+64]<<4, ql[l+32] = L[l+32] | L[l+96]<<4,
    qh[l] = top 2 bits of L[l], L[l+32], L[l+64], L[l+96] at bits 0,2,4,6."""
    ql, qh = bytearray(128), bytearray(64)
    for h in range(2):
        j = 128 * h
        for l in range(32):
            q1, q2, q3, q4 = (L[j + l + o] for o in (0, 32, 64, 96))
            ql[64 * h + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            ql[64 * h + l + 32] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            qh[32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    return q6_block(d16, ql, qh, sc)


@pytest.mark.parametrize("seed", range(20))
def test_q4_k_unpack_and_dequant_against_encoder(seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, 256).tolist()
    sc = rng.integers(0, 64, 8).tolist()
    m = rng.integers(0, 64, 8).tolist()
    d16, dm16 = (int(v) for v in rng.integers(0, 0x7C00, 2))
    blk = encode_q4_k(d16, dm16, sc, m, q)
    uq, usc, um, ud, udm = O.unpack_q4_k(blk)
    assert uq.tolist() == q and usc.tolist() == sc and um.tolist() == m
    d = np.float16(np.uint16(d16).view(np.float16)).astype(np.float64)
    dm = np.float16(np.uint16(dm16).view(np.float16)).astype(np.float64)
    assert ud[0] == d and udm[0] == dm
    # f32 dequant = one rounding of the exact value (quants.rs:129-131)
    exact = np.array([d * sc[e // 32] * q[e] - dm * m[e // 32] for e in range(256)])
    assert np.array_equal(O.dequantize(O.Q4_K, blk, 256), exact.astype(np.float32))


@pytest.mark.parametrize("seed", range(20))
def test_q6_k_unpack_and_dequant_against_encoder(seed):
    rng = np.random.default_rng(100 + seed)
    L = rng.integers(0, 64, 256).tolist()
    sc = rng.integers(-128, 128, 16).tolist()
    d16 = int(rng.integers(0, 0x7C00))
    blk = encode_q6_k(d16, sc, L)
    uq, usc, ud = O.unpack_q6_k(blk)
    assert uq.tolist() == L and usc.tolist() == sc
    d = np.uint16(d16).view(np.float16).astype(np.float64)
    exact = np.array([d * sc[e // 16] * (L[e] - 32) for e in range(256)])
    deq = O.dequantize(O.Q6_K, blk, 256)
    assert np.array_equal(deq.astype(np.float64), exact)  # exact in f32 (quants.rs:170)


@pytest.mark.parametrize("seed", range(10))
def test_q8_0_unpack_and_dequant_closed_form(seed):
    rng = np.random.default_rng(200 + seed)
    q = rng.integers(-128, 128, 64).astype(np.int8)
    d16 = rng.integers(0, 0x7C00, 2).astype(np.uint16)
    blk = b"".join(int(d16[i]).to_bytes(2, "little") + q[32 * i:32 * i + 32].tobytes() for i in range(2))
    uq, ud = O.unpack_q8_0(blk)
    assert np.array_equal(uq, q)
    d = d16.view(np.float16).astype(np.float64)
    exact = np.repeat(d, 32) * q.astype(np.float64)
    assert np.array_equal(O.dequantize(O.Q8_0, blk, 64).astype(np.float64), exact)


@pytest.mark.parametrize("dtype", [O.Q4_K, O.Q6_K, O.Q8_0])
def test_dot_equals_exactly_rounded_sum_on_integer_products(dtype):
    """With d = 1 and integer x, every product is an integer < 2^53 and the
    f64 sum is exact in any order: dot must equal numpy's exact integer dot
    of x with the dequantized row (pins the map, not the tree)."""
    import uq.synth as S
    rng = np.random.default_rng(7)
    n = 1024
    w = S.blocks(dtype, n // S.BLOCK_ELEMS[dtype], rng).reshape(-1, S.BLOCK_BYTES[dtype])
    if dtype == O.Q6_K:
        w[:, 208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    else:
        w[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        if dtype == O.Q4_K:
            w[:, 2:4] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    w = w.reshape(-1)
    x = rng.integers(-1000, 1000, n).astype(np.float32)
    deq = O.dequantize(dtype, w, n).astype(np.int64)
    exp = float(np.dot(x.astype(np.int64), deq))
    dot = {O.Q4_K: O.dot_q4_k, O.Q6_K: O.dot_q6_k, O.Q8_0: O.dot_q8_0}[dtype]
    assert dot(x, w) == exp


# ---------------------------------------------------------------- real-byte pins

def _pins():
    with open(os.path.join(GOLDEN, "reference_pins.json")) as f:
        return json.load(f)


def test_ornith_decode_pin():  # quants.rs:1154-1222 against gguf-py values
    fx = _pins()
    i = np.arange(256)
    xp = ((i * 7919) % 1009).astype(np.float32) / np.float32(1009.0) - np.float32(0.5)
    xa = ((i * 31 + 17) % 257).astype(np.float32) / np.float32(257.0) - np.float32(0.5)
    hot7, hot200 = np.zeros(256, np.float32), np.zeros(256, np.float32)
    hot7[7] = hot200[200] = 1.0
    for case in fx["cases"]:
        blk = bytes(fx["blocks"][case["block"]]["bytes"])
        dot = O.dot_q6_k if len(blk) == 210 else O.dot_q4_k
        for x, key in ((xp, "dot_x_pattern"), (xa, "dot_x_alt"), (hot7, "w7"), (hot200, "w200")):
            assert abs(dot(x, blk) - case[key]) < fx["tolerance"], (case["block"], key)


# ---------------------------------------------------------------- a10: Q8_K

def test_nearest_int_replicates_ggml_magic():  # quants.rs:954-965
    for v, e in [(0.0, 0), (2.5, 2), (3.5, 4), (-3.5, -4), (126.7, 127), (-126.7, -127),
                 (0.5, 0), (1.5, 2)]:
        assert O.nearest_int(v) == e


def test_nearest_int_is_round_half_even_on_working_range():
    v = np.linspace(-127.5, 127.5, 20001, dtype=np.float32)
    v = np.concatenate([v, np.arange(-127, 128, dtype=np.float32) + np.float32(0.5)])
    got = np.array([O.nearest_int(float(t)) for t in v])
    assert np.array_equal(got, np.rint(v).astype(np.int64))


def test_quantize_q8_k_hand_block_and_zero_block():  # quants.rs:967-1000
    x = np.zeros(256, np.float32)
    x[0] = 1.0
    q = O.quantize_q8_k(x)
    assert len(q) == 1 and q[0]["qs"][0] == -127 and np.all(q[0]["qs"][1:] == 0)
    assert q[0]["bsums"][0] == -127 and np.all(q[0]["bsums"][1:] == 0)
    assert q[0]["d"] == np.float32(1.0) / np.float32(-127.0)
    x[0] = -1.0
    q = O.quantize_q8_k(x)
    assert q[0]["qs"][0] == -127 and q[0]["d"] == np.float32(1.0) / np.float32(127.0)
    q = O.quantize_q8_k(np.zeros(256, np.float32))
    assert q[0]["d"] == 0.0 and np.all(q[0]["qs"] == 0)
    two = np.zeros(512, np.float32)
    two[256] = 2.0
    q = O.quantize_q8_k(two)
    assert len(q) == 2 and q[0]["d"] == 0.0 and q[1]["qs"][0] == -127


@pytest.mark.parametrize("seed", range(5))
def test_quantize_q8_k_against_numpy_formulation(seed):
    """Independent statement: signed max = first index of max |x|; iscale =
    -127/max in f32; qs = min(127, rint(f32(iscale*x))); bsums over 16;
    d = 1/iscale. Includes a tie for max |x| (first index must win)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(1024).astype(np.float32)
    x[300], x[301] = 5.0, -5.0   # tie: +5 comes first -> max = +5
    x[700], x[650] = -4.0, 4.0   # tie: +4 comes first (650 < 700)
    q = O.quantize_q8_k(x)
    for b in range(4):
        c = x[256 * b: 256 * b + 256]
        mx = c[int(np.argmax(np.abs(c)))]
        isc = np.float32(-127.0) / mx
        qs = np.minimum(127, np.rint((isc * c).astype(np.float32))).astype(np.int8)
        assert np.array_equal(q[b]["qs"], qs)
        assert np.array_equal(q[b]["bsums"], qs.astype(np.int32).reshape(16, 16).sum(1))
        assert q[b]["d"] == np.float32(1.0) / isc


# ---------------------------------------------------------------- a11/a12: Q8_K dots

def test_dot_q4_k_q8_k_hand_values():  # quants.rs:1002-1021
    scales = bytearray(12)
    scales[0], scales[4] = 1, 3
    qs = bytearray(128)
    qs[0] = 0x01
    blk = q4_block(F16_ONE, F16_TWO, scales, qs)
    x = np.zeros(256, np.float32)
    x[0] = 127.0
    assert O.dot_q4_k_q8_k(O.quantize_q8_k(x), blk) == -635.0


def test_dot_q6_k_q8_k_hand_values():  # quants.rs:1023-1057
    ql = [0] * 128
    ql[0] = 0x01
    sc = [0] * 16
    sc[0] = 1
    x = np.zeros(256, np.float32)
    x[0] = 127.0
    assert O.dot_q6_k_q8_k(O.quantize_q8_k(x), q6_block(F16_ONE, ql, [0] * 64, sc)) == -3937.0
    ql = [0] * 128
    ql[32] = 0x01
    sc = [0] * 16
    sc[2] = -1
    x = np.zeros(256, np.float32)
    x[32] = 127.0
    assert O.dot_q6_k_q8_k(O.quantize_q8_k(x), q6_block(F16_ONE, ql, [0] * 64, sc)) == 3937.0


def test_q8k_dots_close_to_exact_dots():  # quants.rs:1059-1083
    fx = _pins()
    i = np.arange(256)
    xp = ((i * 7919) % 1009).astype(np.float32) / np.float32(1009.0) - np.float32(0.5)
    q = O.quantize_q8_k(xp)
    for name, v in fx["blocks"].items():
        blk = bytes(v["bytes"])
        if len(blk) == 144:
            assert abs(O.dot_q4_k(xp, blk) - O.dot_q4_k_q8_k(q, blk)) < 0.5
        else:
            assert abs(O.dot_q6_k(xp, blk) - O.dot_q6_k_q8_k(q, blk)) < 0.5


@pytest.mark.parametrize("dtype", [O.Q4_K, O.Q6_K])
def test_q8k_dot_exact_when_every_operation_is_exact(dtype):
    """x integer in [-127,127] with one element at 127: Q8_K quantization is
    the identity up to sign (iscale = -1, d = -1), d/dmin are powers of two,
    so every f32 operation of the generic kernel is exact and the result must
    equal numpy's exact integer dot with the dequantized weights (pins maps,
    signs and the min term; summation order cannot show here)."""
    import uq.synth as S
    rng = np.random.default_rng(11)
    nb = 8
    w = S.blocks(dtype, nb, rng).reshape(nb, -1)
    one, two = (np.frombuffer(np.float16(v).tobytes(), np.uint8) for v in (0.25, 0.5))
    if dtype == O.Q4_K:
        w[:, 0:2], w[:, 2:4] = one, two
    else:
        w[:, 208:210] = one
    w = w.reshape(-1)
    x = rng.integers(-126, 127, 256 * nb).astype(np.float32)
    x[::256] = 127.0
    deq = O.dequantize(dtype, w, 256 * nb).astype(np.float64)
    exp = float(np.dot(x.astype(np.float64), deq))
    q = O.quantize_q8_k(x)
    got = (O.dot_q4_k_q8_k if dtype == O.Q4_K else O.dot_q6_k_q8_k)(q, w)
    assert got == exp


def test_dot_q4_k_q8_k_epilogue_order():
    """quants.rs:310, :355-358: s = ((sumf + sums[0]) + sums[1]) + ... with
    sumf holding every block's dmin subtraction. Block A puts 122,895,360 in
    lane 0; block B puts -122,895,360 in sumf and +1 in lane 1. Only the
    documented order keeps the 1 (adding lanes first loses it to rounding:
    ulp(1.2e8) = 8)."""
    f16 = lambda v: int(np.float16(v).view(np.uint16))
    sa = bytearray(12)
    sa[0] = 63                      # sc0 = 63, m0 = 0
    qa = bytearray(128)
    qa[0] = 15                      # element 0 nibble 15
    blk_a = q4_block(f16(1024.0), 0, sa, qa)
    sb = bytearray(12)
    sb[0], sb[4] = 1, 63            # sc0 = 1, m0 = 63
    qb = bytearray(128)
    qb[1] = 1                       # element 1 nibble 1
    blk_b = q4_block(f16(1.0), f16(15240.0), sb, qb)
    x = np.zeros(512, np.float32)
    x[0], x[256], x[257] = 127.0, 127.0, 1.0
    xq = O.quantize_q8_k(x)
    assert xq[0]["d"] == -1.0 and xq[1]["d"] == -1.0
    assert O.dot_q4_k_q8_k(xq, blk_a + blk_b) == 1.0


# ---------------------------------------------------------------- a9/a13: gemv checks

def test_gemv_quant_error_classes():  # quants.rs:430-452, :482-505
    w = np.zeros(144 * 2, np.uint8)
    x = np.zeros(256, np.float32)
    with pytest.raises(O.OracleError) as e:
        O.gemv_quant(np.zeros(3, np.float32), x, w, 256, 2, O.Q4_K)
    assert e.value.kind == "LEN"
    with pytest.raises(O.OracleError) as e:
        O.gemv_quant(np.zeros(2, np.float32), x[:100], w, 256, 2, O.Q4_K)
    assert e.value.kind == "LEN"
    with pytest.raises(O.OracleError) as e:
        O.gemv_quant(np.zeros(2, np.float32), x, w, 128, 2, O.Q4_K)
    assert e.value.kind == "BLOCK_MULTIPLE"
    with pytest.raises(O.OracleError) as e:
        O.gemv_quant(np.zeros(2, np.float32), x, w, 256, 2, O.F16)
    assert e.value.kind == "DTYPE"
    with pytest.raises(O.OracleError) as e:
        O.gemv_quant(np.zeros(2, np.float32), x, w[:-1], 256, 2, O.Q4_K)
    assert e.value.kind == "LEN"
    with pytest.raises(O.OracleError) as e:
        O.gemv_quant_q8k(np.zeros(2, np.float32), x, w, 256, 2, O.F32)
    assert e.value.kind == "DTYPE"


def test_gemv_quant_rows_and_longer_x():
    """gemv_quant = per-row dot over x[..dim_in] (quants.rs:453-465); x may
    be longer than dim_in (:431)."""
    import uq.synth as S
    w = S.weights(O.Q6_K, 5, 512, seed=3)
    x = S.activations(600, seed=3)
    out = np.zeros(5, np.float32)
    O.gemv_quant(out, x, w, 512, 5, O.Q6_K)
    for j in range(5):
        assert out[j] == np.float32(O.dot_q6_k(x[:512], w[j * 420:(j + 1) * 420]))
    out_mt = np.zeros(5, np.float32)
    O.gemv_quant(out_mt, x, w, 512, 5, O.Q6_K, nthreads=3)
    assert np.array_equal(out, out_mt)


def test_row_bytes_sizes_are_exact():  # min_forward.rs:270-282
    assert O.row_bytes(O.F32, 4096) == 16384
    assert O.row_bytes(O.Q4_K, 4096) == 16 * 144
    assert O.row_bytes(O.Q6_K, 4096) == 16 * 210
    assert O.row_bytes(O.Q8_0, 64) == 2 * 34
    assert O.row_bytes(O.Q4_K, 4097) == 0 and O.row_bytes(O.Q8_0, 33) == 0


# ---------------------------------------------------------------- a15: swiglu/silu

def test_swiglu_hand_values():  # kernels.rs:595-611
    out = O.swiglu([0.0, 3.0], [7.0, 0.0])
    assert out[0] == 0.0 and out[1] == 0.0
    out = O.swiglu([1.0], [2.0])
    t = 1.0
    e = np.float32(t * (1.0 / (1.0 + math.exp(-t))) * 2.0)
    assert out[0] == e and abs(out[0] - 1.4621172) < 1e-6


def test_silu_hand_values():  # kernels.rs:626-650
    assert np.all(O.silu([0.0, 0.0, 0.0]) == 0.0)
    t = 1.0
    assert O.silu([1.0])[0] == np.float32(t / (1.0 + math.exp(-t)))


def test_swiglu_close_to_f64_formula():
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(4096) * 30).astype(np.float32)
    u = (rng.standard_normal(4096) * 30).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(O.swiglu(g, u), ref, rtol=3e-7, atol=1e-30)


@pytest.mark.parametrize("dtype", [O.Q4_K, O.Q6_K, O.Q8_0])
def test_exact_f64_weights_reproduce_gemv_quant(dtype):
    """tests/helpers.exact_weights_f64 (used as the reference of the GEMM
    tests at full size) against the oracle's gemv_quant: the f64 product
    X @ W.T equals gemv_quant row for row after rounding to f32, except where
    the two f64 summation orders straddle an f32 rounding boundary (at most
    1 ulp, and rarely). Also across an adversarial x with huge and tiny
    entries, and with Q6_K scales over the full int8 range."""
    from helpers import exact_weights_f64
    K, N = 1024, 96
    rng = np.random.default_rng(dtype)
    bb, be = O.BLOCK_BYTES[dtype], O.BLOCK_ELEMS[dtype]
    b = rng.integers(0, 256, size=(N * K // be, bb), dtype=np.uint8)  # scales over the full int8 range
    dpos = {O.Q4_K: (0, 2), O.Q6_K: (208,), O.Q8_0: (0,)}[dtype]
    for p in dpos:  # finite f16 scales
        b[:, p:p + 2] = np.abs(rng.normal(0, 2e-3, b.shape[0])).astype(np.float16).view(np.uint8).reshape(-1, 2)
    w = b.reshape(-1)
    W = exact_weights_f64(dtype, w, N, K)
    for x in (rng.standard_normal(K).astype(np.float32),
              (rng.standard_normal(K) * 10.0 ** rng.uniform(-6, 6, K)).astype(np.float32)):
        ref = np.zeros(N, np.float32)
        O.gemv_quant(ref, x, w, K, N, dtype)
        y = (W @ x.astype(np.float64)).astype(np.float32)
        ulp = np.abs(y.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
        assert int(ulp.max()) <= 1 and int((ulp > 0).sum()) <= 2, (int(ulp.max()), int((ulp > 0).sum()))
