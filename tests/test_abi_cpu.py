"""libuq.so without a GPU: it loads, exports every symbol include/*.h
declare, refuses bad arguments with the reference's panic classes before
touching a device, and fails loudly (no CPU fallback) when no GPU exists."""
import glob
import os
import re

import ctypes as C

import numpy as np
import pytest

import uq

INCLUDE = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include")


def declared_functions():
    names = set()
    for h in sorted(glob.glob(os.path.join(INCLUDE, "*.h"))):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(uq_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    L = uq.lib()
    names = declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) == set(uq.SIGNATURES), set(names) ^ set(uq.SIGNATURES)


def test_row_bytes():  # min_forward.rs:270-282
    assert uq.row_bytes(uq.DType.F32, 4096) == 16384
    assert uq.row_bytes(uq.DType.Q4K, 4096) == 16 * 144
    assert uq.row_bytes(uq.DType.Q6K, 4096) == 16 * 210
    assert uq.row_bytes(uq.DType.Q8_0, 64) == 2 * 34
    assert uq.row_bytes(uq.DType.Q4K, 4097) == 0 and uq.row_bytes(uq.DType.Q8_0, 33) == 0


def _raises(kind, fn, *a):
    with pytest.raises(uq.UqError) as e:
        fn(*a)
    assert e.value.kind == kind, str(e.value)


def test_gemv_quant_argument_errors_mirror_reference_panics():  # quants.rs:430-452
    w = np.zeros(144 * 2, np.uint8)
    x = np.zeros(256, np.float32)
    _raises("LEN", uq.gemv_quant, np.zeros(3, np.float32), x, w, 256, 2, uq.DType.Q4K)
    _raises("LEN", uq.gemv_quant, np.zeros(2, np.float32), x[:100], w, 256, 2, uq.DType.Q4K)
    _raises("BLOCK_MULTIPLE", uq.gemv_quant, np.zeros(2, np.float32), x, w, 128, 2, uq.DType.Q4K)
    _raises("DTYPE", uq.gemv_quant, np.zeros(2, np.float32), x, w, 256, 2, uq.DType.F16)
    _raises("LEN", uq.gemv_quant, np.zeros(2, np.float32), x, w[:-1], 256, 2, uq.DType.Q4K)
    _raises("BLOCK_MULTIPLE", uq.gemv_quant, np.zeros(1, np.float32), x, np.zeros(34, np.uint8), 16, 1,
            uq.DType.Q8_0)


def test_gemv_quant_q8k_argument_errors():  # quants.rs:482-505
    w = np.zeros(144 * 2, np.uint8)
    x = np.zeros(256, np.float32)
    _raises("DTYPE", uq.gemv_quant_q8k, np.zeros(2, np.float32), x, w, 256, 2, uq.DType.F32)
    _raises("DTYPE", uq.gemv_quant_q8k, np.zeros(2, np.float32), x, w, 256, 2, uq.DType.Q8_0)
    _raises("BLOCK_MULTIPLE", uq.gemv_quant_q8k, np.zeros(2, np.float32), x, w, 128, 2, uq.DType.Q4K)
    _raises("LEN", uq.gemv_quant_q8k, np.zeros(1, np.float32), x, w, 256, 2, uq.DType.Q4K)


def test_dequant_and_quantize_argument_errors():  # quants.rs:535-539, :251-255
    _raises("LEN", uq.dequantize_q4_k, np.zeros(512, np.float32), np.zeros(144, np.uint8))
    _raises("LEN", uq.dequantize_q4_k, np.zeros(300, np.float32), np.zeros(144, np.uint8))
    _raises("LEN", uq.dequantize_q6_k, np.zeros(256, np.float32), np.zeros(209, np.uint8))
    _raises("BLOCK_MULTIPLE", uq.quantize_q8_k, np.zeros(100, np.float32))


def test_empty_shapes_need_no_device():
    out = np.zeros(0, np.float32)
    uq.gemv_quant(out, np.zeros(256, np.float32), np.zeros(0, np.uint8), 256, 0, uq.DType.Q4K)
    out = np.full(3, 7.0, np.float32)
    uq.gemv_quant(out, np.zeros(0, np.float32), np.zeros(0, np.uint8), 0, 3, uq.DType.Q4K)
    assert np.all(out == 0.0)  # empty dot = 0 (pairwise_sum of nothing, kernels.rs:41)


@pytest.mark.skipif(uq.device_count() > 0, reason="a GPU is present")
def test_compute_fails_loudly_without_gpu():
    x = np.zeros(256, np.float32)
    w = np.zeros(144, np.uint8)
    _raises("NO_DEVICE", uq.gemv_quant, np.zeros(1, np.float32), x, w, 256, 1, uq.DType.Q4K)
    _raises("NO_DEVICE", uq.Weights, w, uq.DType.Q4K, 256, 1)


def test_gemv_batch_argument_errors():
    """uq_gemv_batch validates before touching a device: null tables, count
    above UQ_GEMV_BATCH_MAX, invalid handles."""
    L = uq.lib()
    P = C.c_void_p
    hs = (P * 9)()
    ys = (P * 9)()
    assert uq.STATUS[L.uq_gemv_batch(None, ys, 1, None, None)] == "ARG"
    assert uq.STATUS[L.uq_gemv_batch(hs, None, 1, None, None)] == "ARG"
    assert L.uq_gemv_batch(hs, ys, 0, None, None) == 0  # nothing to do
    assert uq.STATUS[L.uq_gemv_batch(hs, ys, 9, None, None)] == "ARG"
    assert uq.STATUS[L.uq_gemv_batch(hs, ys, 2, None, None)] == "ARG"  # null handles


def test_ops_argument_errors_mirror_reference_panics():  # kernels.rs asserts, before any device work
    from uq import ops
    f = np.zeros(4, np.float32)
    L = uq.lib()
    P = lambda a: a.ctypes.data_as(C.c_void_p)
    assert uq.STATUS[L.uq_rmsnorm(P(f), 3, P(f), 4, P(f), 4, 0.0)] == "LEN"
    assert uq.STATUS[L.uq_rmsnorm(P(f), 4, P(f), 4, P(f), 3, 0.0)] == "LEN"
    assert uq.STATUS[L.uq_softmax(P(f), 3, P(f), 4, 1.0)] == "LEN"
    assert uq.STATUS[L.uq_sigmoid(P(f), 3, P(f), 4)] == "LEN"
    assert uq.STATUS[L.uq_l2_norm_rows(P(f), 4, 3, 1e-6)] == "LEN"
    assert uq.STATUS[L.uq_ssm_conv(P(f), 2, P(f), 3, P(f), 4, 2, 2)] == "LEN"       # len(x) % channels
    assert uq.STATUS[L.uq_ssm_conv(P(f), 2, P(f), 4, P(f), 4, 4, 2)] == "LEN"       # window shorter than kernel
    assert uq.STATUS[L.uq_ssm_conv(P(f), 2, P(f), 4, P(f), 3, 2, 2)] == "LEN"       # len(kernel)
    assert uq.STATUS[L.uq_ssm_conv(P(f), 3, P(f), 4, P(f), 4, 2, 2)] == "LEN"       # len(out)
    assert uq.STATUS[L.uq_gdn_fused_step(P(f), 4, P(f), 2, P(f), 2, P(f), 1, P(f), 2, 0.0, 1.0, 1.0)] == "LEN"
    assert uq.STATUS[L.uq_gdn_fused_step(P(f), 3, P(f), 2, P(f), 2, P(f), 2, P(f), 2, 0.0, 1.0, 1.0)] == "LEN"
    assert uq.STATUS[L.uq_rope_llama(P(f), 3, P(f), 4, 1)] == "LEN"
    assert uq.STATUS[L.uq_rope_neox(P(f), 4, P(f), 1, 1)] == "LEN"
    assert uq.STATUS[L.uq_rope_imrope(P(f), 4, 3, 0.5, 1)] == "LEN"
    assert uq.STATUS[L.uq_rope_imrope(P(f), 4, 6, 0.5, 1)] == "LEN"
    # attention: shape limits, then the slice lengths
    g = np.zeros(256, np.float32)
    assert uq.STATUS[L.uq_attn_decode(P(g), 128, P(g), 128, P(g), 64, P(g), 64, 1, 2, 3, 64, 1.0)] == "ARG"  # 2 % 3
    assert uq.STATUS[L.uq_attn_decode(P(g), 96, P(g), 96, P(g), 96, P(g), 96, 1, 1, 1, 96, 1.0)] == "ARG"   # head_dim
    assert uq.STATUS[L.uq_attn_decode(P(g), 64, P(g), 64, P(g), 64, P(g), 64, 0, 1, 1, 64, 1.0)] == "ARG"   # n_ctx 0
    assert uq.STATUS[L.uq_attn_decode(P(g), 64, P(g), 32, P(g), 64, P(g), 64, 1, 1, 1, 64, 1.0)] == "LEN"   # len(q)
    assert uq.STATUS[L.uq_attn_decode(P(g), 64, P(g), 64, P(g), 63, P(g), 64, 1, 1, 1, 64, 1.0)] == "LEN"   # len(k)
    assert uq.STATUS[L.uq_attn_decode(P(g), 64, P(g), 64, P(g), 64, P(g), 127, 2, 1, 1, 64, 1.0)] == "LEN"  # len(v)
    assert uq.STATUS[L.uq_attn_decode(P(g), 63, P(g), 64, P(g), 64, P(g), 64, 1, 1, 1, 64, 1.0)] == "LEN"   # len(out)
    assert uq.STATUS[L.uq_attn_decode_d(P(g), P(g), P(g), P(g), P(g), 1, 18, 2, 64, 1.0, None)] == "ARG"  # group 9
    # matmul_f32_acc: len(a), len(b), len(acc) in that order; gelu; embedding_lookup
    assert uq.STATUS[L.uq_matmul_f32_acc(P(f), 4, P(f), 5, P(f), 7, 2, 3, 2)] == "LEN"
    assert uq.STATUS[L.uq_matmul_f32_acc(P(f), 3, P(g), 6, P(g), 7, 2, 3, 2)] == "LEN"
    assert uq.STATUS[L.uq_matmul_f32_acc(P(f), 3, P(g), 6, P(g), 6, 2, 3, 2)] == "LEN"
    assert uq.STATUS[L.uq_gelu_tanh(P(f), 3, P(f), 4)] == "LEN"
    ids = np.array([0, 99], np.uint32)
    assert uq.STATUS[L.uq_embedding_lookup(P(f), 4, P(g), 7, P(ids), 2, 2)] == "LEN"    # len(table) % dim
    assert uq.STATUS[L.uq_embedding_lookup(P(f), 3, P(g), 6, P(ids), 2, 2)] == "LEN"    # len(out)
    assert uq.STATUS[L.uq_embedding_lookup(P(f), 4, P(g), 6, P(ids), 2, 2)] == "TOKEN"  # id 99 past 3 rows
    assert uq.STATUS[L.uq_embedding_lookup_d(P(f), P(g), 6, P(ids), 2, 2, None)] == "TOKEN"
    if uq.device_count() == 0:
        with pytest.raises(uq.UqError) as e:
            ops.rmsnorm(f, f, 1e-6)
        assert e.value.kind == "NO_DEVICE"
