"""Per-layer non-linear ops of libuq (include/uq_ops.h), named after
crates/unltd-tensor/src/kernels.rs. Host forms take numpy arrays and return
new arrays (the in-place reference functions return the updated copy);
device forms (suffix _d) take uq.DeviceArray buffers and a stream."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import DeviceArray, _check, _f32, _ptr, lib


def rmsnorm(x, w, eps: float) -> np.ndarray:
    """kernels.rs:61-78"""
    x, w = _f32(x), _f32(w)
    out = np.zeros(len(x), np.float32)
    _check(lib().uq_rmsnorm(_ptr(out), len(out), _ptr(x), len(x), _ptr(w), len(w), eps))
    return out


def rmsnorm_d(d_out: DeviceArray, d_x: DeviceArray, d_w: DeviceArray, n: int, rows: int, eps: float, stream=None):
    _check(lib().uq_rmsnorm_d(d_out.ptr, d_x.ptr, d_w.ptr, n, rows, eps, stream))


def l2_norm_rows(data, dim: int, eps: float) -> np.ndarray:
    """kernels.rs:236-256"""
    d = _f32(data).copy()
    _check(lib().uq_l2_norm_rows(_ptr(d), len(d), dim, eps))
    return d


def l2_norm_rows_d(d_data: DeviceArray, length: int, dim: int, eps: float, stream=None):
    _check(lib().uq_l2_norm_rows_d(d_data.ptr, length, dim, eps, stream))


def softmax(x, scale: float) -> np.ndarray:
    """kernels.rs:157-168"""
    x = _f32(x)
    out = np.zeros(len(x), np.float32)
    _check(lib().uq_softmax(_ptr(out), len(out), _ptr(x), len(x), scale))
    return out


def softmax_d(d_out: DeviceArray, d_x: DeviceArray, n: int, rows: int, scale: float, stream=None):
    _check(lib().uq_softmax_d(d_out.ptr, d_x.ptr, n, rows, scale, stream))


def _unary(name, x):
    x = _f32(x)
    out = np.zeros(len(x), np.float32)
    _check(getattr(lib(), name)(_ptr(out), len(out), _ptr(x), len(x)))
    return out


def sigmoid(x) -> np.ndarray:
    return _unary("uq_sigmoid", x)


def silu(x) -> np.ndarray:
    return _unary("uq_silu", x)


def softplus(x) -> np.ndarray:
    return _unary("uq_softplus", x)


def gelu_tanh(x) -> np.ndarray:
    """kernels.rs:185-194"""
    return _unary("uq_gelu_tanh", x)


def unary_d(name: str, d_out: DeviceArray, d_x: DeviceArray, n: int, stream=None):
    """name: sigmoid, silu, softplus or gelu_tanh"""
    _check(getattr(lib(), f"uq_{name}_d")(d_out.ptr, d_x.ptr, n, stream))


def ssm_conv(x, kernel, d_conv: int, channels: int) -> np.ndarray:
    """kernels.rs:265-305"""
    x, k = _f32(x), _f32(kernel)
    n_t = len(x) // channels - (d_conv - 1) if channels else 0
    out = np.zeros(max(n_t, 0) * channels, np.float32)
    _check(lib().uq_ssm_conv(_ptr(out), len(out), _ptr(x), len(x), _ptr(k), len(k), d_conv, channels))
    return out


def ssm_conv_d(d_out: DeviceArray, d_x: DeviceArray, x_len: int, d_kernel: DeviceArray, d_conv: int, channels: int,
               stream=None):
    _check(lib().uq_ssm_conv_d(d_out.ptr, d_x.ptr, x_len, d_kernel.ptr, d_conv, channels, stream))


def gdn_fused_step(state, q, k, v, gate: float, beta: float, scale: float):
    """kernels.rs:316-375; returns (new state, out)"""
    st = _f32(state).copy()
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros(len(q), np.float32)
    _check(lib().uq_gdn_fused_step(_ptr(st), len(st), _ptr(out), len(out), _ptr(q), len(q), _ptr(k), len(k),
                                   _ptr(v), len(v), gate, beta, scale))
    return st, out


def gdn_fused_step_d(d_state, d_out, d_q, d_k, d_v, d_gate, d_beta, dim: int, heads: int, scale: float,
                     stream=None):
    _check(lib().uq_gdn_fused_step_d(d_state.ptr, d_out.ptr, d_q.ptr, d_k.ptr, d_v.ptr, d_gate.ptr, d_beta.ptr, dim,
                                     heads, scale, stream))


def rope_llama(x, freqs, pos: int) -> np.ndarray:
    """kernels.rs:109-125"""
    y, f = _f32(x).copy(), _f32(freqs)
    _check(lib().uq_rope_llama(_ptr(y), len(y), _ptr(f), len(f), pos))
    return y


def rope_neox(x, freqs, pos: int) -> np.ndarray:
    """kernels.rs:131-148"""
    y, f = _f32(x).copy(), _f32(freqs)
    _check(lib().uq_rope_neox(_ptr(y), len(y), _ptr(f), len(f), pos))
    return y


def rope_d(kind: str, d_x: DeviceArray, n: int, rows: int, d_freqs: DeviceArray, pos: int, stream=None):
    """kind: llama or neox"""
    _check(getattr(lib(), f"uq_rope_{kind}_d")(d_x.ptr, n, rows, d_freqs.ptr, pos, stream))


def rope_imrope(x, n_rot: int, theta_scale: float, pos: int) -> np.ndarray:
    """kernels.rs:381-400"""
    y = _f32(x).copy()
    _check(lib().uq_rope_imrope(_ptr(y), len(y), n_rot, theta_scale, pos))
    return y


def rope_imrope_d(d_x: DeviceArray, n: int, rows: int, n_rot: int, theta_scale: float, pos: int, stream=None):
    _check(lib().uq_rope_imrope_d(d_x.ptr, n, rows, n_rot, theta_scale, pos, stream))


def attn_decode(q, k_cache, v_cache, n_ctx: int, n_head: int, n_head_kv: int, head_dim: int,
                kq_scale: float) -> np.ndarray:
    """qwen35_forward.rs:639-671 (step 5 of attn_layer): the attention of one
    decode position over n_ctx cached positions; returns out [n_head*head_dim]."""
    q, kc, vc = _f32(q), _f32(k_cache), _f32(v_cache)
    out = np.zeros(n_head * head_dim, np.float32)
    _check(lib().uq_attn_decode(_ptr(out), len(out), _ptr(q), len(q), _ptr(kc), len(kc), _ptr(vc), len(vc),
                                n_ctx, n_head, n_head_kv, head_dim, kq_scale))
    return out


def attn_decode_d(d_out: DeviceArray, d_soft: DeviceArray, d_q: DeviceArray, d_k_cache: DeviceArray,
                  d_v_cache: DeviceArray, n_ctx: int, n_head: int, n_head_kv: int, head_dim: int, kq_scale: float,
                  stream=None):
    _check(lib().uq_attn_decode_d(d_out.ptr, d_soft.ptr, d_q.ptr, d_k_cache.ptr, d_v_cache.ptr, n_ctx, n_head,
                                  n_head_kv, head_dim, kq_scale, stream))


def matmul_f32_acc(acc, a, b, m: int, k: int, n: int) -> np.ndarray:
    """kernels.rs:87-101; returns the updated copy of acc"""
    out, a, b = _f32(acc).copy(), _f32(a), _f32(b)
    _check(lib().uq_matmul_f32_acc(_ptr(out), len(out), _ptr(a), len(a), _ptr(b), len(b), m, k, n))
    return out


def matmul_f32_acc_d(d_acc: DeviceArray, d_a: DeviceArray, d_b: DeviceArray, m: int, k: int, n: int, stream=None):
    _check(lib().uq_matmul_f32_acc_d(d_acc.ptr, d_a.ptr, d_b.ptr, m, k, n, stream))


def embedding_lookup(table, ids, dim: int) -> np.ndarray:
    """kernels.rs:402-422"""
    t = _f32(table)
    ids = np.ascontiguousarray(ids, np.uint32)
    out = np.zeros(len(ids) * dim, np.float32)
    _check(lib().uq_embedding_lookup(_ptr(out), len(out), _ptr(t), len(t), _ptr(ids), len(ids), dim))
    return out


def embedding_lookup_d(d_out: DeviceArray, d_table: DeviceArray, table_len: int, ids, dim: int, stream=None):
    ids = np.ascontiguousarray(ids, np.uint32)
    _check(lib().uq_embedding_lookup_d(d_out.ptr, d_table.ptr, table_len, _ptr(ids), len(ids), dim, stream))

