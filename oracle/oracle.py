"""ctypes wrapper of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: the oracle the GPU kernels are compared against.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module. Function names mirror the reference's
(crates/unltd-tensor/src/quants.rs, kernels.rs); reference panics surface as
OracleError with the same status classes as the product library.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
QK_K = 256
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, Q8_0: 34}
BLOCK_ELEMS = {Q4_K: 256, Q6_K: 256, Q8_0: 32}
STATUS = {1: "LEN", 2: "BLOCK_MULTIPLE", 3: "DTYPE", 4: "ALLOC"}

Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i4", (16,))],
                     align=True)


class OracleError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: {STATUS.get(code, code)}")
        self.code = code
        self.kind = STATUS.get(code, str(code))


def build() -> str:
    """Compile liboracle.so with its Makefile (gcc)."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liboracle.so"], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        S = C.c_size_t
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_f16_to_f32.restype = C.c_float
        L.or_scale_min_k4.argtypes = [P, C.c_int, P, P]
        L.or_pairwise_sum_f64.argtypes = [P, S, P]
        L.or_pairwise_sum_f64.restype = C.c_double
        for n in ("or_dot_f32", "or_dot_q4_k", "or_dot_q6_k", "or_dot_q8_0"):
            getattr(L, n).argtypes = [P, P, S]
            getattr(L, n).restype = C.c_double
        L.or_row_bytes.argtypes = [C.c_int, S]
        L.or_row_bytes.restype = S
        for n in ("or_gemv_quant", "or_gemv_quant_q8k"):
            getattr(L, n).argtypes = [P, S, P, S, P, S, S, S, C.c_int]
            getattr(L, n).restype = C.c_int
        for n in ("or_gemv_quant_mt", "or_gemv_quant_q8k_mt"):
            getattr(L, n).argtypes = [P, S, P, S, P, S, S, S, C.c_int, C.c_int]
            getattr(L, n).restype = C.c_int
        L.or_nearest_int.argtypes = [C.c_float]
        L.or_nearest_int.restype = C.c_int32
        L.or_quantize_q8_k.argtypes = [P, P, S]
        L.or_quantize_q8_k.restype = C.c_int
        for n in ("or_dot_q4_k_q8_k", "or_dot_q6_k_q8_k"):
            getattr(L, n).argtypes = [P, S, P]
            getattr(L, n).restype = C.c_float
        for n in ("or_dequantize_q4_k", "or_dequantize_q6_k", "or_dequantize_q8_0"):
            getattr(L, n).argtypes = [P, S, P, S]
            getattr(L, n).restype = C.c_int
        L.or_unpack_q4_k.argtypes = [P, S, P, P, P, P, P]
        L.or_unpack_q6_k.argtypes = [P, S, P, P, P]
        L.or_unpack_q8_0.argtypes = [P, S, P, P]
        L.or_swiglu.argtypes = [P, P, P, S]
        L.or_silu.argtypes = [P, P, S]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _check(rc: int, what: str):
    if rc != 0:
        raise OracleError(rc, what)


def f16_to_f32(h: int) -> np.float32:
    return np.float32(lib().or_f16_to_f32(h))


def f16_to_f32_array(h: np.ndarray) -> np.ndarray:
    f = lib().or_f16_to_f32
    return np.array([f(int(v)) for v in h.ravel()], dtype=np.float32).reshape(h.shape)


def scale_min_k4(s: bytes, g: int):
    s = np.frombuffer(bytes(s), dtype=np.uint8)
    sc = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().or_scale_min_k4(_p(s), g, _p(sc), _p(m))
    return int(sc[0]), int(m[0])


def pairwise_sum_f64(v) -> float:
    v = np.ascontiguousarray(v, dtype=np.float64)
    scratch = np.empty(max(len(v), 1), np.float64)
    return lib().or_pairwise_sum_f64(_p(v), len(v), _p(scratch))


def _u8(w) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(w), dtype=np.uint8)
                                if isinstance(w, (bytes, bytearray)) else w, dtype=np.uint8)


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def dot_f32(x, w) -> float:
    x, w = _f32(x), _f32(w)
    assert len(x) == len(w)
    return lib().or_dot_f32(_p(x), _p(w), len(x))


def dot_q4_k(x, w) -> float:
    x, w = _f32(x), _u8(w)
    assert len(x) % QK_K == 0 and len(w) == len(x) // QK_K * 144
    return lib().or_dot_q4_k(_p(x), _p(w), len(x))


def dot_q6_k(x, w) -> float:
    x, w = _f32(x), _u8(w)
    assert len(x) % QK_K == 0 and len(w) == len(x) // QK_K * 210
    return lib().or_dot_q6_k(_p(x), _p(w), len(x))


def dot_q8_0(x, w) -> float:
    x, w = _f32(x), _u8(w)
    assert len(x) % 32 == 0 and len(w) == len(x) // 32 * 34
    return lib().or_dot_q8_0(_p(x), _p(w), len(x))


def row_bytes(dtype: int, n: int) -> int:
    return lib().or_row_bytes(dtype, n)


def gemv_quant(out: np.ndarray, x, w, dim_in: int, dim_out: int, dtype: int,
               nthreads: int = 1) -> None:
    x, w = _f32(x), _u8(w)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    rc = lib().or_gemv_quant_mt(_p(out), out.size, _p(x), x.size, _p(w), w.size,
                                dim_in, dim_out, dtype, nthreads)
    _check(rc, "gemv_quant")


def gemv_quant_q8k(out: np.ndarray, x, w, dim_in: int, dim_out: int, dtype: int,
                   nthreads: int = 1) -> None:
    x, w = _f32(x), _u8(w)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    rc = lib().or_gemv_quant_q8k_mt(_p(out), out.size, _p(x), x.size, _p(w), w.size,
                                    dim_in, dim_out, dtype, nthreads)
    _check(rc, "gemv_quant_q8k")


def nearest_int(f: float) -> int:
    return lib().or_nearest_int(f)


def quantize_q8_k(x) -> np.ndarray:
    x = _f32(x)
    out = np.zeros(max(len(x) // QK_K, 1), dtype=Q8K_DTYPE)
    _check(lib().or_quantize_q8_k(_p(out), _p(x), len(x)), "quantize_q8_k")
    return out[: len(x) // QK_K]


def dot_q4_k_q8_k(xq: np.ndarray, w) -> float:
    w = _u8(w)
    assert len(w) == len(xq) * 144
    return float(np.float32(lib().or_dot_q4_k_q8_k(_p(xq), len(xq), _p(w))))


def dot_q6_k_q8_k(xq: np.ndarray, w) -> float:
    w = _u8(w)
    assert len(w) == len(xq) * 210
    return float(np.float32(lib().or_dot_q6_k_q8_k(_p(xq), len(xq), _p(w))))


def _dequant(fn, out: np.ndarray, w, what):
    w = _u8(w)
    _check(getattr(lib(), fn)(_p(out), out.size, _p(w), w.size), what)


def dequantize_q4_k(out: np.ndarray, w) -> None:
    _dequant("or_dequantize_q4_k", out, w, "dequantize_q4_k")


def dequantize_q6_k(out: np.ndarray, w) -> None:
    _dequant("or_dequantize_q6_k", out, w, "dequantize_q6_k")


def dequantize_q8_0(out: np.ndarray, w) -> None:
    _dequant("or_dequantize_q8_0", out, w, "dequantize_q8_0")


def dequantize(dtype: int, w, n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    {Q4_K: dequantize_q4_k, Q6_K: dequantize_q6_k, Q8_0: dequantize_q8_0}[dtype](out, w)
    return out


def unpack_q4_k(w):
    w = _u8(w)
    nb = len(w) // 144
    q = np.zeros(nb * 256, np.uint8)
    sc = np.zeros(nb * 8, np.uint8)
    m = np.zeros(nb * 8, np.uint8)
    d = np.zeros(nb, np.float32)
    dmin = np.zeros(nb, np.float32)
    lib().or_unpack_q4_k(_p(w), nb, _p(q), _p(sc), _p(m), _p(d), _p(dmin))
    return q, sc, m, d, dmin


def unpack_q6_k(w):
    w = _u8(w)
    nb = len(w) // 210
    q = np.zeros(nb * 256, np.uint8)
    sc = np.zeros(nb * 16, np.int8)
    d = np.zeros(nb, np.float32)
    lib().or_unpack_q6_k(_p(w), nb, _p(q), _p(sc), _p(d))
    return q, sc, d


def unpack_q8_0(w):
    w = _u8(w)
    nb = len(w) // 34
    q = np.zeros(nb * 32, np.int8)
    d = np.zeros(nb, np.float32)
    lib().or_unpack_q8_0(_p(w), nb, _p(q), _p(d))
    return q, d


def swiglu(gate, up) -> np.ndarray:
    g, u = _f32(gate), _f32(up)
    out = np.zeros(len(g), np.float32)
    lib().or_swiglu(_p(out), _p(g), _p(u), len(g))
    return out


def silu(x) -> np.ndarray:
    x = _f32(x)
    out = np.zeros(len(x), np.float32)
    lib().or_silu(_p(out), _p(x), len(x))
    return out


# ------------------------------------------------ per-layer ops (oracle_ops.c)

def _fn(name, argtypes, restype=C.c_int):
    f = getattr(lib(), name)
    f.argtypes = argtypes
    f.restype = restype
    return f


def _ok(rc, what):
    if rc != 0:
        raise ValueError(f"{what}: oracle status {rc}")


_P, _S = C.c_void_p, C.c_size_t


def rmsnorm(x, w, eps: float) -> np.ndarray:
    """kernels.rs:61-78"""
    x, w = _f32(x), _f32(w)
    out = np.zeros(len(x), np.float32)
    _ok(_fn("or_rmsnorm", [_P, _P, _P, _S, C.c_float])(_p(out), _p(x), _p(w), len(x), eps), "rmsnorm")
    return out


def l2_norm_rows(data, dim: int, eps: float) -> np.ndarray:
    """kernels.rs:236-256 (returns a normalised copy)"""
    d = _f32(data).copy()
    _ok(_fn("or_l2_norm_rows", [_P, _S, _S, C.c_float])(_p(d), len(d), dim, eps), "l2_norm_rows")
    return d


def softmax(x, scale: float) -> np.ndarray:
    """kernels.rs:157-168"""
    x = _f32(x)
    out = np.zeros(len(x), np.float32)
    _ok(_fn("or_softmax", [_P, _P, _S, C.c_float])(_p(out), _p(x), len(x), scale), "softmax")
    return out


def sigmoid(x) -> np.ndarray:
    x = _f32(x)
    out = np.zeros(len(x), np.float32)
    _fn("or_sigmoid", [_P, _P, _S], None)(_p(out), _p(x), len(x))
    return out


def softplus(x) -> np.ndarray:
    x = _f32(x)
    out = np.zeros(len(x), np.float32)
    _fn("or_softplus", [_P, _P, _S], None)(_p(out), _p(x), len(x))
    return out


def ssm_conv(x, kernel, d_conv: int, channels: int) -> np.ndarray:
    """kernels.rs:265-305; out[t*channels + c]"""
    x, k = _f32(x), _f32(kernel)
    n_t = len(x) // channels - (d_conv - 1)
    out = np.zeros(max(n_t, 0) * channels, np.float32)
    _ok(_fn("or_ssm_conv", [_P, _S, _P, _S, _P, _S, _S, _S])(_p(out), len(out), _p(x), len(x), _p(k), len(k),
                                                             d_conv, channels), "ssm_conv")
    return out


def gdn_fused_step(state, q, k, v, gate: float, beta: float, scale: float):
    """kernels.rs:316-375; returns (new state, out)"""
    st = _f32(state).copy()
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros(len(q), np.float32)
    _ok(_fn("or_gdn_fused_step", [_P, _P, _P, _P, _P, _S, C.c_float, C.c_float, C.c_float])(
        _p(st), _p(out), _p(q), _p(k), _p(v), len(q), gate, beta, scale), "gdn_fused_step")
    return st, out


def rope_llama(x, freqs, pos: int) -> np.ndarray:
    """kernels.rs:109-125 (returns a rotated copy)"""
    y, f = _f32(x).copy(), _f32(freqs)
    _ok(_fn("or_rope_llama", [_P, _S, _P, _S, _S])(_p(y), len(y), _p(f), len(f), pos), "rope_llama")
    return y


def rope_neox(x, freqs, pos: int) -> np.ndarray:
    """kernels.rs:131-148"""
    y, f = _f32(x).copy(), _f32(freqs)
    _ok(_fn("or_rope_neox", [_P, _S, _P, _S, _S])(_p(y), len(y), _p(f), len(f), pos), "rope_neox")
    return y


def matmul_f32_acc(acc, a, b, m: int, k: int, n: int) -> np.ndarray:
    """kernels.rs:87-101; returns the updated copy of acc"""
    out, a, b = _f32(acc).copy(), _f32(a), _f32(b)
    _ok(_fn("or_matmul_f32_acc", [_P, _P, _P, _S, _S, _S])(_p(out), _p(a), _p(b), m, k, n), "matmul_f32_acc")
    return out


def gelu_tanh(x) -> np.ndarray:
    """kernels.rs:185-194"""
    x = _f32(x)
    out = np.zeros(len(x), np.float32)
    _fn("or_gelu_tanh", [_P, _P, _S], None)(_p(out), _p(x), len(x))
    return out


def embedding_lookup(table, ids, dim: int) -> np.ndarray:
    """kernels.rs:402-422"""
    t = _f32(table)
    ids = np.ascontiguousarray(ids, np.uint32)
    out = np.zeros(len(ids) * dim, np.float32)
    _ok(_fn("or_embedding_lookup", [_P, _S, _P, _S, _P, _S, _S])(_p(out), len(out), _p(t), len(t), _p(ids), len(ids),
                                                                 dim), "embedding_lookup")
    return out


def attn_decode(q, k_cache, v_cache, n_ctx: int, n_head: int, n_head_kv: int, hd: int, kq_scale: float):
    """qwen35_forward.rs:639-671; returns (out [n_head*hd], soft [n_head*n_ctx])"""
    q, kc, vc = _f32(q), _f32(k_cache), _f32(v_cache)
    out = np.zeros(n_head * hd, np.float32)
    soft = np.zeros(n_head * n_ctx, np.float32)
    _ok(_fn("or_attn_decode", [_P, _P, _P, _P, _P, _S, _S, _S, _S, C.c_float])(
        _p(out), _p(soft), _p(q), _p(kc), _p(vc), n_ctx, n_head, n_head_kv, hd, kq_scale), "attn_decode")
    return out, soft


def rope_imrope(x, n_rot: int, theta_scale: float, pos: int) -> np.ndarray:
    """kernels.rs:381-400"""
    y = _f32(x).copy()
    _ok(_fn("or_rope_imrope", [_P, _S, _S, C.c_double, _S])(_p(y), len(y), n_rot, theta_scale, pos), "rope_imrope")
    return y


# ------------------------------------------------ one decode layer
# Qwen35Forward::recr_layer, attn_layer and ffn
# (crates/unltd-generation/src/qwen35_forward.rs:333-768), step for step,
# composed from the functions above. cfg carries the uq_qwen35_dims field
# names; w maps a projection name to (bytes, dtype) and a vector name to an
# f32 array. The f32 element-wise additions and products are numpy float32
# operations (each one IEEE rounding, as the reference's).

def _q8k(w, x, dim_in: int, dim_out: int, nthreads: int) -> np.ndarray:
    out = np.zeros(dim_out, np.float32)
    gemv_quant_q8k(out, x, w[0], dim_in, dim_out, w[1], nthreads=nthreads)
    return out


def layer_ffn(cfg, w, residual, nodes: dict, nthreads: int = 1) -> np.ndarray:
    """ffn (qwen35_forward.rs:713-768): f = ffn_down . swiglu(ffn_gate . p, ffn_up . p),
    p = rmsnorm(residual, post_attention_norm)."""
    n, nff = cfg.n_embd, cfg.n_ff
    p = rmsnorm(residual, w["post_attention_norm"], cfg.rms_eps)
    g = _q8k(w["ffn_gate"], p, n, nff, nthreads)
    u = _q8k(w["ffn_up"], p, n, nff, nthreads)
    sw = swiglu(g, u)
    f = _q8k(w["ffn_down"], sw, nff, n, nthreads)
    nodes.update(post_norm=p, ffn_gate=g, ffn_up=u, ffn_swiglu=sw, ffn_out=f)
    return f


def recr_layer(cfg, w, ring: np.ndarray, state: np.ndarray, x_in, nthreads: int = 1):
    """recr_layer (qwen35_forward.rs:333-543) for one token. ring
    [conv_kernel - 1][channels] and state [n_v][hd][hd] are updated in place,
    as the session's conv ring and GDN state. Returns (l_out, nodes)."""
    n, eps = cfg.n_embd, cfg.rms_eps
    nqk, nv, hd, ck = cfg.n_qk_heads, cfg.n_v_heads, cfg.head_dim_linear, cfg.conv_kernel
    ch = 2 * nqk * hd + nv * hd
    x_in = _f32(x_in)
    nodes = {}
    x = rmsnorm(x_in, w["attn_norm"], eps)                                 # :352-360
    qkv = _q8k(w["attn_qkv"], x, n, ch, nthreads)                          # :363-372
    z = _q8k(w["attn_gate"], x, n, nv * hd, nthreads)                      # :373-381
    beta_raw = _q8k(w["ssm_beta"], x, n, nv, nthreads)                     # :386-394
    alpha = _q8k(w["ssm_alpha"], x, n, nv, nthreads)                       # :395-403
    beta = sigmoid(beta_raw)                                               # :405
    sp = softplus(alpha + w["ssm_dt_bias"])                                # :413-416
    gate = sp * w["ssm_a"]                                                 # :417-419
    win = np.concatenate([ring.reshape(-1), qkv])                          # :427-431
    kernel = np.ascontiguousarray(_f32(w["ssm_conv1d"]).reshape(ch, ck).T).reshape(-1)  # :441-446
    conv = ssm_conv(win, kernel, ck, ch)                                   # :447
    ring[:-1] = ring[1:].copy()                                            # :449-450
    ring[-1] = qkv
    mix = silu(conv)                                                       # :454
    qc = l2_norm_rows(mix[:nqk * hd], hd, eps)                             # :463
    kc = l2_norm_rows(mix[nqk * hd:2 * nqk * hd], hd, eps)                 # :464
    vc = mix[2 * nqk * hd:]
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))                      # :472
    out = np.zeros(nv * hd, np.float32)
    for h in range(nv):                                                    # :474-491
        qk = h % nqk
        st, o = gdn_fused_step(state[h].reshape(-1), qc[qk * hd:(qk + 1) * hd], kc[qk * hd:(qk + 1) * hd],
                               vc[h * hd:(h + 1) * hd], float(gate[h]), float(beta[h]), float(scale))
        state[h] = st.reshape(hd, hd)
        out[h * hd:(h + 1) * hd] = o
    y = np.concatenate([rmsnorm(out[h * hd:(h + 1) * hd], w["ssm_norm"], eps) for h in range(nv)])  # :495-505
    y = y * silu(z)                                                        # :507-511
    attn_out = _q8k(w["ssm_out"], y, nv * hd, n, nthreads)                 # :514-521
    residual = x_in + attn_out                                             # :524-527
    nodes.update(attn_norm=x, qkv=qkv, z=z, beta_raw=beta_raw, alpha=alpha, beta=beta, a_softplus=sp, gate=gate,
                 conv_raw=conv, conv_silu=np.concatenate([qc, kc, vc]), gdn_out=out, final=y, attn_out=attn_out,
                 residual=residual)
    f = layer_ffn(cfg, w, residual, nodes, nthreads)                      # :530
    return residual + f, nodes                                             # :533-536


def attn_layer(cfg, w, k_cache: np.ndarray, v_cache: np.ndarray, pos: int, x_in, nthreads: int = 1):
    """attn_layer (qwen35_forward.rs:546-710) for one token at pos. The
    caches [n_ctx][n_head_kv * head_dim] get row pos. Returns (l_out, nodes)."""
    n, eps = cfg.n_embd, cfg.rms_eps
    nh, nkv, hd = cfg.n_head, cfg.n_head_kv, cfg.head_dim
    x_in = _f32(x_in)
    nodes = {}
    x = rmsnorm(x_in, w["attn_norm"], eps)                                 # :563-571
    qfull = _q8k(w["attn_q"], x, n, 2 * nh * hd, nthreads)                 # :573-582
    q = np.concatenate([rmsnorm(qfull[2 * h * hd:2 * h * hd + hd], w["attn_q_norm"], eps) for h in range(nh)])
    gate = np.concatenate([qfull[2 * h * hd + hd:2 * (h + 1) * hd] for h in range(nh)])  # :583-600
    k = _q8k(w["attn_k"], x, n, nkv * hd, nthreads)                        # :603-610
    kn = np.concatenate([rmsnorm(k[i * hd:(i + 1) * hd], w["attn_k_norm"], eps) for i in range(nkv)])  # :611-623
    v = _q8k(w["attn_v"], x, n, nkv * hd, nthreads)                        # :625-632
    q = np.concatenate([rope_imrope(q[h * hd:(h + 1) * hd], cfg.n_rot, cfg.theta_scale, pos)
                        for h in range(nh)])                               # :634-639
    kn = np.concatenate([rope_imrope(kn[i * hd:(i + 1) * hd], cfg.n_rot, cfg.theta_scale, pos)
                         for i in range(nkv)])                             # :640-642
    k_cache[pos] = kn                                                      # :643-645
    v_cache[pos] = v
    attn, soft = attn_decode(q, k_cache[:pos + 1], v_cache[:pos + 1], pos + 1, nh, nkv, hd, cfg.kq_scale)  # :647-675
    gated = attn * sigmoid(gate)                                           # :677-684
    attn_out = _q8k(w["attn_output"], gated, nh * hd, n, nthreads)         # :686-693
    residual = x_in + attn_out                                             # :696-699
    nodes.update(attn_norm=x, qfull=qfull, k_raw=k, q=q, k_row=kn, v_row=v, attn=attn, soft=soft, gated=gated,
                 attn_out=attn_out, residual=residual)
    f = layer_ffn(cfg, w, residual, nodes, nthreads)                      # :700
    return residual + f, nodes                                             # :701-704
