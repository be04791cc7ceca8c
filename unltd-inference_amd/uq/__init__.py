"""ctypes binding of libuq.so (include/uq.h), named after unltd-tensor's API.

Host-pointer mirrors (gemv_quant, gemv_quant_q8k, quantize_q8_k,
dequantize_q4_k, ...) take numpy arrays where the reference takes slices and
raise UqError where the reference panics (crates/unltd-tensor/src/quants.rs).
The device-resident API is exposed as Weights / DeviceArray / gemv / gemv_q8k /
gemm / ffn_swiglu. Loading the library needs the HIP runtime but no GPU; every
compute call needs an MI355X (gfx950) and fails loudly without one.
"""
from __future__ import annotations

import ctypes as C
import enum
import os

import numpy as np

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "libuq.so")
EMU_PATH = os.path.join(_PKG, "libuq_emu.so")


class DType(enum.IntEnum):
    """ggml type ids (min_forward.rs:39-48)."""
    F32 = 0
    F16 = 1
    Q8_0 = 8
    Q4K = 12
    Q6K = 14


STATUS = {0: "OK", 1: "LEN", 2: "BLOCK_MULTIPLE", 3: "DTYPE", 4: "ARG", 5: "HIP", 6: "NO_DEVICE", 7: "TOKEN",
          8: "FILE", 9: "MAGIC", 10: "VERSION", 11: "TENSOR_BOUNDS", 12: "TENSOR_OVERLAP", 13: "TENSOR_ALIGN",
          14: "GGML_TYPE", 15: "MISSING_TENSOR", 16: "ELEMENT_COUNT", 17: "IO"}

Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i4", (16,))], align=True)
assert Q8K_DTYPE.itemsize == 324


class UqError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code
        self.kind = STATUS.get(code, str(code))


_lib = None

# (name, argtypes) of every symbol include/uq.h declares
_P, _S, _I = C.c_void_p, C.c_size_t, C.c_int
SIGNATURES = {
    "uq_last_error": ([], C.c_char_p),
    "uq_status_name": ([_I], C.c_char_p),
    "uq_row_bytes": ([_I, _S], _S),
    "uq_gemv_quant": ([_P, _S, _P, _S, _P, _S, _S, _S, _I], _I),
    "uq_gemv_quant_q8k": ([_P, _S, _P, _S, _P, _S, _S, _S, _I], _I),
    "uq_quantize_q8_k": ([_P, _S, _P, _S], _I),
    "uq_dequantize_q4_k": ([_P, _S, _P, _S], _I),
    "uq_dequantize_q6_k": ([_P, _S, _P, _S], _I),
    "uq_dequantize_q8_0": ([_P, _S, _P, _S], _I),
    "uq_unpack_q4_k": ([_P, _S, _P, _P, _P, _P, _P], _I),
    "uq_unpack_q6_k": ([_P, _S, _P, _P, _P], _I),
    "uq_unpack_q8_0": ([_P, _S, _P, _P], _I),
    "uq_f16_to_f32": ([_P, _P, _S], _I),
    "uq_swiglu": ([_P, _P, _P, _S], _I),
    "uq_weights_upload": ([C.POINTER(_P), _P, _S, _I, _S, _S], _I),
    "uq_weights_free": ([_P], _I),
    "uq_weights_info": ([_P, C.POINTER(_I), C.POINTER(_S), C.POINTER(_S), C.POINTER(_S)], _I),
    "uq_gemv": ([_P, _P, _P, _P], _I),
    "uq_gemv_batch": ([_P, _P, _S, _P, _P], _I),
    "uq_gemv_q8k_batch": ([_P, _P, _S, _P, _P], _I),
    "uq_ffn_swiglu_q8k": ([_P, _P, _P, _P, _P, _P, _P, _P, _P], _I),
    "uq_swiglu_d": ([_P, _P, _P, _S, _P], _I),
    "uq_gemv_q8k": ([_P, _P, _P, _P], _I),
    "uq_gemm": ([_P, _S, _P, _P, _P], _I),
    "uq_gemm_static": ([_P, _S, _P, _P, _P], _I),
    "uq_gemm_q8k": ([_P, _S, _P, _P, _P], _I),
    "uq_gemm_q8k_batch": ([_P, _P, _S, _S, _P, _P], _I),
    "uq_ffn_swiglu": ([_P, _P, _P, _P, _P, _P, _P], _I),
    "uq_dequantize": ([_P, _P, _P], _I),
    "uq_embed": ([_P, _P, _S, _P, _P], _I),
    "uq_device_count": ([C.POINTER(_I)], _I),
    "uq_device_name": ([C.c_char_p, _S], _I),
    "uq_malloc": ([C.POINTER(_P), _S], _I),
    "uq_free": ([_P], _I),
    "uq_memcpy_htod": ([_P, _P, _S, _P], _I),
    "uq_memcpy_dtoh": ([_P, _P, _S, _P], _I),
    "uq_memcpy_dtod": ([_P, _P, _S, _P], _I),
    "uq_stream_synchronize": ([_P], _I),
    # include/uq_gguf.h
    "uq_gguf_open": ([C.c_char_p, C.POINTER(_P)], _I),
    "uq_gguf_parse": ([_P, _S, C.POINTER(_P)], _I),
    "uq_gguf_close": ([_P], _I),
    "uq_gguf_header": ([_P, _P, _P, _P, _P, _P], _I),
    "uq_gguf_tensor_at": ([_P, C.c_uint64, _P], _I),
    "uq_gguf_find": ([_P, C.c_char_p, _P], _I),
    "uq_gguf_tensor_bytes": ([_P, C.c_char_p, _P, _P], _I),
    "uq_gguf_tensor_checked": ([_P, C.c_char_p, C.c_uint64, _P, _P], _I),
    "uq_gguf_check": ([_P, C.c_char_p, C.c_uint64, C.c_uint64, _P], _I),
    "uq_gguf_upload": ([_P, C.c_char_p, C.POINTER(_P)], _I),
    "uq_gguf_kv_at": ([_P, C.c_uint64, _P], _I),
    "uq_gguf_kv_find": ([_P, C.c_char_p, _P], _I),
    "uq_gguf_kv_string": ([_P, C.c_uint64, C.c_uint64, _P, _P], _I),
    "uq_gguf_type_blocksize": ([C.c_uint32, _P, _P], _I),
    "uq_gguf_type_name": ([C.c_uint32, C.c_char_p, _S], _I),
    # include/uq_ops.h
    "uq_rmsnorm": ([_P, _S, _P, _S, _P, _S, C.c_float], _I),
    "uq_rmsnorm_d": ([_P, _P, _P, _S, _S, C.c_float, _P], _I),
    "uq_l2_norm_rows": ([_P, _S, _S, C.c_float], _I),
    "uq_l2_norm_rows_d": ([_P, _S, _S, C.c_float, _P], _I),
    "uq_softmax": ([_P, _S, _P, _S, C.c_float], _I),
    "uq_softmax_d": ([_P, _P, _S, _S, C.c_float, _P], _I),
    "uq_sigmoid": ([_P, _S, _P, _S], _I),
    "uq_silu": ([_P, _S, _P, _S], _I),
    "uq_softplus": ([_P, _S, _P, _S], _I),
    "uq_sigmoid_d": ([_P, _P, _S, _P], _I),
    "uq_silu_d": ([_P, _P, _S, _P], _I),
    "uq_softplus_d": ([_P, _P, _S, _P], _I),
    "uq_ssm_conv": ([_P, _S, _P, _S, _P, _S, _S, _S], _I),
    "uq_ssm_conv_d": ([_P, _P, _S, _P, _S, _S, _P], _I),
    "uq_gdn_fused_step": ([_P, _S, _P, _S, _P, _S, _P, _S, _P, _S, C.c_float, C.c_float, C.c_float], _I),
    "uq_gdn_fused_step_d": ([_P, _P, _P, _P, _P, _P, _P, _S, _S, C.c_float, _P], _I),
    "uq_rope_llama": ([_P, _S, _P, _S, _S], _I),
    "uq_rope_neox": ([_P, _S, _P, _S, _S], _I),
    "uq_rope_llama_d": ([_P, _S, _S, _P, _S, _P], _I),
    "uq_rope_neox_d": ([_P, _S, _S, _P, _S, _P], _I),
    "uq_rope_imrope": ([_P, _S, _S, C.c_double, _S], _I),
    "uq_rope_imrope_d": ([_P, _S, _S, _S, C.c_double, _S, _P], _I),
    "uq_gelu_tanh": ([_P, _S, _P, _S], _I),
    "uq_gelu_tanh_d": ([_P, _P, _S, _P], _I),
    "uq_matmul_f32_acc": ([_P, _S, _P, _S, _P, _S, _S, _S, _S], _I),
    "uq_matmul_f32_acc_d": ([_P, _P, _P, _S, _S, _S, _P], _I),
    "uq_embedding_lookup": ([_P, _S, _P, _S, _P, _S, _S], _I),
    "uq_embedding_lookup_d": ([_P, _P, _S, _P, _S, _S, _P], _I),
    "uq_attn_decode": ([_P, _S, _P, _S, _P, _S, _P, _S, _S, _S, _S, _S, C.c_float], _I),
    "uq_attn_decode_d": ([_P, _P, _P, _P, _P, _S, _S, _S, _S, C.c_float, _P], _I),
    # include/uq_layer.h (struct arguments by address; uq.layer builds them)
    "uq_layer_ws_floats": ([_P, _S], _S),
    "uq_layer_node_at": ([_P, _S, C.c_int, _P, _P], _I),
    "uq_gdn_layer_step_d": ([_P, _P, _P, _P, _P, _P, _P, _S, _P], _I),
    "uq_attn_layer_step_d": ([_P, _P, _P, _P, _S, _S, _P, _P, _P, _S, _P], _I),
    "uq_layer_prefill_ws_floats": ([_P, _P, _P, _S, _S], _S),
    "uq_gdn_layer_prefill_d": ([_P, _P, _P, _P, _S, _P, _P, _P, _S, _P], _I),
    "uq_attn_layer_prefill_d": ([_P, _P, _P, _P, _S, _S, _S, _P, _P, _P, _S, _P], _I),
}


def lib():
    """Load libuq.so (built by unltd-inference_amd/build.py). No fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run unltd-inference_amd/build.py")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def _check(rc: int):
    if rc != 0:
        raise UqError(rc, lib().uq_last_error().decode("utf-8", "replace"))


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a) -> np.ndarray:
    if isinstance(a, (bytes, bytearray)):
        return np.frombuffer(bytes(a), dtype=np.uint8)
    return np.ascontiguousarray(a).view(np.uint8).reshape(-1)


def row_bytes(dtype: int, dim_in: int) -> int:
    return lib().uq_row_bytes(int(dtype), dim_in)


# ------------------------------------------------------ host-pointer mirrors

def gemv_quant(out: np.ndarray, x, w, dim_in: int, dim_out: int, dtype: int) -> None:
    """quants.rs:422-466 (Q8_0 accepted as well)."""
    x, w = _f32(x), _u8(w)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    _check(lib().uq_gemv_quant(_ptr(out), out.size, _ptr(x), x.size, _ptr(w), w.size,
                               dim_in, dim_out, int(dtype)))


def gemv_quant_q8k(out: np.ndarray, x, w, dim_in: int, dim_out: int, dtype: int) -> None:
    """quants.rs:474-515, bit-exact."""
    x, w = _f32(x), _u8(w)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    _check(lib().uq_gemv_quant_q8k(_ptr(out), out.size, _ptr(x), x.size, _ptr(w), w.size,
                                   dim_in, dim_out, int(dtype)))


def quantize_q8_k(x) -> np.ndarray:
    """quants.rs:250-290, bit-exact; returns an array of Q8K_DTYPE records."""
    x = _f32(x)
    nb = x.size // 256 if x.size % 256 == 0 else 0
    out = np.zeros(max(nb, 1), dtype=Q8K_DTYPE)
    _check(lib().uq_quantize_q8_k(_ptr(out), nb, _ptr(x), x.size))
    return out[:nb]


def _dequant(fn, out, w):
    w = _u8(w)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    _check(getattr(lib(), fn)(_ptr(out), out.size, _ptr(w), w.size))


def dequantize_q4_k(out: np.ndarray, w) -> None:
    """quants.rs:534-567, bit-exact."""
    _dequant("uq_dequantize_q4_k", out, w)


def dequantize_q6_k(out: np.ndarray, w) -> None:
    _dequant("uq_dequantize_q6_k", out, w)


def dequantize_q8_0(out: np.ndarray, w) -> None:
    _dequant("uq_dequantize_q8_0", out, w)


def unpack_q4_k(w):
    w = _u8(w)
    nb = w.size // 144
    q = np.zeros(nb * 256, np.uint8)
    sc, m = np.zeros(nb * 8, np.uint8), np.zeros(nb * 8, np.uint8)
    d, dmin = np.zeros(nb, np.float32), np.zeros(nb, np.float32)
    _check(lib().uq_unpack_q4_k(_ptr(w), nb, _ptr(q), _ptr(sc), _ptr(m), _ptr(d), _ptr(dmin)))
    return q, sc, m, d, dmin


def unpack_q6_k(w):
    w = _u8(w)
    nb = w.size // 210
    q, sc, d = np.zeros(nb * 256, np.uint8), np.zeros(nb * 16, np.int8), np.zeros(nb, np.float32)
    _check(lib().uq_unpack_q6_k(_ptr(w), nb, _ptr(q), _ptr(sc), _ptr(d)))
    return q, sc, d


def unpack_q8_0(w):
    w = _u8(w)
    nb = w.size // 34
    q, d = np.zeros(nb * 32, np.int8), np.zeros(nb, np.float32)
    _check(lib().uq_unpack_q8_0(_ptr(w), nb, _ptr(q), _ptr(d)))
    return q, d


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.zeros(h.size, np.float32)
    _check(lib().uq_f16_to_f32(_ptr(out), _ptr(h), h.size))
    return out


def swiglu(gate, up) -> np.ndarray:
    g, u = _f32(gate), _f32(up)
    out = np.zeros(g.size, np.float32)
    _check(lib().uq_swiglu(_ptr(out), _ptr(g), _ptr(u), g.size))
    return out


# ------------------------------------------------------ device-resident API

class DeviceArray:
    """A float32 / byte buffer in HBM owned by libuq's allocator."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        _check(lib().uq_malloc(C.byref(p), nbytes))
        self.ptr, self.nbytes = p, nbytes

    @classmethod
    def from_numpy(cls, a: np.ndarray, stream=None) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        d.upload(a, stream)
        return d

    def upload(self, a: np.ndarray, stream=None):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _check(lib().uq_memcpy_htod(self.ptr, _ptr(a), a.nbytes, stream))
        if stream is None:
            _check(lib().uq_stream_synchronize(None))

    def download(self, dtype=np.float32, count: int | None = None, stream=None) -> np.ndarray:
        n = self.nbytes // np.dtype(dtype).itemsize if count is None else count
        out = np.empty(n, dtype=dtype)
        _check(lib().uq_memcpy_dtoh(_ptr(out), self.ptr, out.nbytes, stream))
        return out

    def free(self):
        if self.ptr:
            _check(lib().uq_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weights:
    """One GGUF tensor copied to HBM unchanged (uq_weights_upload)."""

    def __init__(self, data, dtype: int, dim_in: int, dim_out: int):
        b = _u8(data)
        h = C.c_void_p()
        _check(lib().uq_weights_upload(C.byref(h), _ptr(b), b.size, int(dtype), dim_in, dim_out))
        self.h, self.dtype, self.dim_in, self.dim_out, self.nbytes = h, int(dtype), dim_in, dim_out, b.size

    @classmethod
    def from_handle(cls, h: C.c_void_p) -> "Weights":
        """Adopt a handle made by the library (e.g. uq_gguf_upload)."""
        self = cls.__new__(cls)
        dt, di, do, nb = C.c_int(), C.c_size_t(), C.c_size_t(), C.c_size_t()
        _check(lib().uq_weights_info(h, C.byref(dt), C.byref(di), C.byref(do), C.byref(nb)))
        self.h, self.dtype, self.dim_in, self.dim_out, self.nbytes = h, dt.value, di.value, do.value, nb.value
        return self

    def free(self):
        if self.h:
            _check(lib().uq_weights_free(self.h))
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def gemv(w: Weights, d_x: DeviceArray, d_y: DeviceArray, stream=None) -> None:
    _check(lib().uq_gemv(w.h, d_x.ptr, d_y.ptr, stream))


GEMV_BATCH_MAX = 8


def gemv_batch(ws, d_x: DeviceArray, d_ys, stream=None) -> None:
    """d_ys[i] = ws[i] . d_x for every i, in one launch (same dtype and dim_in)."""
    n = len(ws)
    hs = (_P * max(n, 1))(*[w.h for w in ws])
    ys = (_P * max(n, 1))(*[y.ptr for y in d_ys])
    _check(lib().uq_gemv_batch(hs, ys, n, d_x.ptr, stream))


def gemv_q8k_batch(ws, d_x: DeviceArray, d_ys, stream=None) -> None:
    """d_ys[i] = gemv_quant_q8k(ws[i], d_x) for every i, in one launch."""
    n = len(ws)
    hs = (_P * max(n, 1))(*[w.h for w in ws])
    ys = (_P * max(n, 1))(*[y.ptr for y in d_ys])
    _check(lib().uq_gemv_q8k_batch(hs, ys, n, d_x.ptr, stream))


def ffn_swiglu_q8k(gate: Weights, up: Weights, down: Weights, d_x: DeviceArray, d_g: DeviceArray,
                   d_u: DeviceArray, d_h: DeviceArray, d_y: DeviceArray, stream=None) -> None:
    _check(lib().uq_ffn_swiglu_q8k(gate.h, up.h, down.h, d_x.ptr, d_g.ptr, d_u.ptr, d_h.ptr, d_y.ptr, stream))


def swiglu_d(d_out: DeviceArray, d_gate: DeviceArray, d_up: DeviceArray, n: int, stream=None) -> None:
    _check(lib().uq_swiglu_d(d_out.ptr, d_gate.ptr, d_up.ptr, n, stream))


def gemv_q8k(w: Weights, d_x: DeviceArray, d_y: DeviceArray, stream=None) -> None:
    _check(lib().uq_gemv_q8k(w.h, d_x.ptr, d_y.ptr, stream))


def gemm(w: Weights, m: int, d_x: DeviceArray, d_y: DeviceArray, stream=None) -> None:
    _check(lib().uq_gemm(w.h, m, d_x.ptr, d_y.ptr, stream))


def gemm_q8k(w: Weights, m: int, d_x: DeviceArray, d_y: DeviceArray, stream=None) -> None:
    """d_y[r] = gemv_quant_q8k(w, d_x[r]) for r < m, bit-exact (uq_gemm_q8k)."""
    _check(lib().uq_gemm_q8k(w.h, m, d_x.ptr, d_y.ptr, stream))


def gemm_q8k_batch(ws, m: int, d_x: DeviceArray, d_ys, stream=None) -> None:
    """d_ys[i][r] = gemv_quant_q8k(ws[i], d_x[r]) for r < m and every i, in one
    launch (same dtype and dim_in; uq_gemm_q8k_batch)."""
    n = len(ws)
    hs = (_P * max(n, 1))(*[w.h for w in ws])
    ys = (_P * max(n, 1))(*[y.ptr for y in d_ys])
    _check(lib().uq_gemm_q8k_batch(hs, ys, n, m, d_x.ptr, stream))


def gemm_static(w: Weights, m: int, d_x: DeviceArray, d_y: DeviceArray, stream=None) -> None:
    """uq_gemm on the library's fixed workspace (allocates nothing)."""
    _check(lib().uq_gemm_static(w.h, m, d_x.ptr, d_y.ptr, stream))


GEMM_SCRATCH_BYTES = 64 << 20


def ffn_swiglu(gate: Weights, up: Weights, down: Weights, d_x: DeviceArray, d_h: DeviceArray,
               d_y: DeviceArray, stream=None) -> None:
    _check(lib().uq_ffn_swiglu(gate.h, up.h, down.h, d_x.ptr, d_h.ptr, d_y.ptr, stream))


def dequantize(w: Weights, d_out: DeviceArray, stream=None) -> None:
    _check(lib().uq_dequantize(w.h, d_out.ptr, stream))


def embed(w: Weights, tokens, d_out: DeviceArray, stream=None) -> None:
    """min_forward.rs:160-184: rows tokens[r] of w into d_out[r*dim_in:]."""
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    _check(lib().uq_embed(w.h, t.ctypes.data_as(C.c_void_p), t.size, d_out.ptr, stream))


def synchronize(stream=None) -> None:
    _check(lib().uq_stream_synchronize(stream))


def device_count() -> int:
    n = C.c_int(0)
    _check(lib().uq_device_count(C.byref(n)))
    return n.value


def device_name() -> str:
    buf = C.create_string_buffer(256)
    _check(lib().uq_device_name(buf, 256))
    return buf.value.decode()


# ------------------------------------------------------ CPU emulation (tests)

_emu = None


def emu():
    """libuq_emu.so: the kernels' per-lane code run on the CPU (test support)."""
    global _emu
    if _emu is None:
        E = C.CDLL(EMU_PATH)
        for n in ("uq_emu_gemv", "uq_emu_gemv_q8k"):
            getattr(E, n).argtypes = [_P, _P, _P, _S, _S, _I]
            getattr(E, n).restype = _I
        E.uq_emu_gemm_q8k.argtypes = [_P, _P, _S, _P, _S, _S, _I]
        E.uq_emu_gemm_q8k.restype = _I
        _emu = E
    return _emu


def emu_gemv(x, w, dim_in: int, dim_out: int, dtype: int, q8k: bool = False) -> np.ndarray:
    x, w = _f32(x), _u8(w)
    y = np.zeros(dim_out, np.float32)
    fn = emu().uq_emu_gemv_q8k if q8k else emu().uq_emu_gemv
    rc = fn(_ptr(y), _ptr(x), _ptr(w), dim_in, dim_out, int(dtype))
    if rc != 0:
        raise ValueError(f"shape not taken by the fast kernels: dtype {dtype}, K {dim_in}")
    return y


def emu_gemm_q8k(X, w, dim_in: int, dim_out: int, dtype: int) -> np.ndarray:
    """uq_gemm_q8k's operand maps and epilogue run on the CPU: Y[m] =
    gemv_quant_q8k(W, X[m])."""
    X, w = _f32(X), _u8(w)
    M = X.size // dim_in
    Y = np.zeros(M * dim_out, np.float32)
    rc = emu().uq_emu_gemm_q8k(_ptr(Y), _ptr(X), M, _ptr(w), dim_in, dim_out, int(dtype))
    if rc != 0:
        raise ValueError(f"uq_gemm_q8k takes Q4_K / Q6_K with K a multiple of 256: dtype {dtype}, K {dim_in}")
    return Y.reshape(M, dim_out)
