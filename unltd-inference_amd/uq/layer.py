"""Device-resident Qwen3.5 layers of libuq (include/uq_layer.h): one token
through a GatedDeltaNet layer (Qwen35Forward::recr_layer,
qwen35_forward.rs:333-543) or a full-attention layer (attn_layer,
:546-710), each with its FFN, on device buffers and a stream; and the
prefill forms, n tokens in one call with the results of n steps."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from . import DeviceArray, Weights, _check, lib

NODES = ["attn_norm", "z", "beta_raw", "alpha", "beta", "a_softplus", "gate", "conv_raw", "conv_silu", "gdn_out",
         "final", "qfull", "k_raw", "q", "attn", "gated", "attn_out", "residual", "post_norm", "ffn_gate", "ffn_up",
         "ffn_swiglu", "ffn_out", "soft"]


class Dims(C.Structure):
    """uq_qwen35_dims"""
    _fields_ = [("n_embd", C.c_size_t), ("n_ff", C.c_size_t), ("n_qk_heads", C.c_size_t),
                ("n_v_heads", C.c_size_t), ("head_dim_linear", C.c_size_t), ("conv_kernel", C.c_size_t),
                ("n_head", C.c_size_t), ("n_head_kv", C.c_size_t), ("head_dim", C.c_size_t),
                ("n_rot", C.c_size_t), ("theta_scale", C.c_double), ("kq_scale", C.c_float),
                ("rms_eps", C.c_float)]

    @property
    def channels(self) -> int:
        return 2 * self.n_qk_heads * self.head_dim_linear + self.n_v_heads * self.head_dim_linear


class _GdnW(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("attn_qkv", "attn_gate", "ssm_beta", "ssm_alpha", "ssm_out", "ffn_gate",
                                          "ffn_up", "ffn_down", "attn_norm", "ssm_dt_bias", "ssm_a", "ssm_conv1d",
                                          "ssm_norm", "post_attention_norm")]


class _AttnW(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                                          "ffn_down", "attn_norm", "attn_q_norm", "attn_k_norm",
                                          "post_attention_norm")]


def ws_floats(d: Dims, n_ctx_max: int = 0) -> int:
    return lib().uq_layer_ws_floats(C.addressof(d), n_ctx_max)


def node_at(d: Dims, node: str, n_ctx_max: int = 0) -> tuple[int, int]:
    """(offset, count) in floats of a node in the workspace."""
    off, cnt = C.c_size_t(), C.c_size_t()
    _check(lib().uq_layer_node_at(C.addressof(d), n_ctx_max, NODES.index(node), C.addressof(off),
                                  C.addressof(cnt)))
    return off.value, cnt.value


@dataclass
class GdnWeights:
    attn_qkv: Weights
    attn_gate: Weights
    ssm_beta: Weights
    ssm_alpha: Weights
    ssm_out: Weights
    ffn_gate: Weights
    ffn_up: Weights
    ffn_down: Weights
    attn_norm: DeviceArray
    ssm_dt_bias: DeviceArray
    ssm_a: DeviceArray
    ssm_conv1d: DeviceArray   # GGUF layout [channels][conv_kernel]
    ssm_norm: DeviceArray
    post_attention_norm: DeviceArray

    def _c(self):
        return _GdnW(*[getattr(self, f[0]).h if isinstance(getattr(self, f[0]), Weights) else getattr(self, f[0]).ptr
                       for f in _GdnW._fields_])


@dataclass
class AttnWeights:
    attn_q: Weights
    attn_k: Weights
    attn_v: Weights
    attn_output: Weights
    ffn_gate: Weights
    ffn_up: Weights
    ffn_down: Weights
    attn_norm: DeviceArray
    attn_q_norm: DeviceArray
    attn_k_norm: DeviceArray
    post_attention_norm: DeviceArray

    def _c(self):
        return _AttnW(*[getattr(self, f[0]).h if isinstance(getattr(self, f[0]), Weights) else getattr(self, f[0]).ptr
                        for f in _AttnW._fields_])


def gdn_step(d: Dims, w: GdnWeights, conv_win: DeviceArray, state: DeviceArray, x_in: DeviceArray,
             l_out: DeviceArray, ws: DeviceArray, stream=None) -> None:
    """uq_gdn_layer_step_d"""
    cw = w._c()
    _check(lib().uq_gdn_layer_step_d(C.addressof(d), C.addressof(cw), conv_win.ptr, state.ptr, x_in.ptr, l_out.ptr,
                                     ws.ptr, ws.nbytes // 4, stream))


def attn_step(d: Dims, w: AttnWeights, k_cache: DeviceArray, v_cache: DeviceArray, n_ctx_max: int, pos: int,
              x_in: DeviceArray, l_out: DeviceArray, ws: DeviceArray, stream=None) -> None:
    """uq_attn_layer_step_d"""
    cw = w._c()
    _check(lib().uq_attn_layer_step_d(C.addressof(d), C.addressof(cw), k_cache.ptr, v_cache.ptr, n_ctx_max, pos,
                                      x_in.ptr, l_out.ptr, ws.ptr, ws.nbytes // 4, stream))


def prefill_ws_floats(d: Dims, n_tokens: int, gdn: GdnWeights | None = None, attn: AttnWeights | None = None,
                      n_ctx_max: int = 0) -> int:
    """uq_layer_prefill_ws_floats: floats of a prefill workspace for n_tokens."""
    g = gdn._c() if gdn is not None else None
    a = attn._c() if attn is not None else None
    return lib().uq_layer_prefill_ws_floats(C.addressof(d), C.addressof(g) if g is not None else None,
                                            C.addressof(a) if a is not None else None, n_ctx_max, n_tokens)


def gdn_prefill(d: Dims, w: GdnWeights, conv_win: DeviceArray, state: DeviceArray, n_tokens: int, x_in: DeviceArray,
                l_out: DeviceArray, ws: DeviceArray, stream=None) -> None:
    """uq_gdn_layer_prefill_d: x_in, l_out are [n_tokens][n_embd]"""
    cw = w._c()
    _check(lib().uq_gdn_layer_prefill_d(C.addressof(d), C.addressof(cw), conv_win.ptr, state.ptr, n_tokens, x_in.ptr,
                                        l_out.ptr, ws.ptr, ws.nbytes // 4, stream))


def attn_prefill(d: Dims, w: AttnWeights, k_cache: DeviceArray, v_cache: DeviceArray, n_ctx_max: int, pos0: int,
                 n_tokens: int, x_in: DeviceArray, l_out: DeviceArray, ws: DeviceArray, stream=None) -> None:
    """uq_attn_layer_prefill_d: positions pos0 .. pos0 + n_tokens - 1"""
    cw = w._c()
    _check(lib().uq_attn_layer_prefill_d(C.addressof(d), C.addressof(cw), k_cache.ptr, v_cache.ptr, n_ctx_max, pos0,
                                         n_tokens, x_in.ptr, l_out.ptr, ws.ptr, ws.nbytes // 4, stream))
