"""GGUF reader and loader of libuq (include/uq_gguf.h), named after the
reference's unltd-model-loader API: GgufReader (gguf.rs:283-350),
MappedWeights (weights.rs:23-96) and the tensor check of
Qwen35Forward::open (qwen35_forward.rs:109-128).

    g = Gguf.open(path)           # MappedWeights::open
    g.get_str("general.architecture")
    g.tensor_checked("blk.0.ffn_up.weight", n_embd * n_ff)
    g.check("blk.0.ffn_down.weight", n_ff * n_embd, [DType.Q4K, DType.Q6K])
    w = g.upload("blk.0.ffn_up.weight")   # a uq.Weights in HBM, bytes unchanged

Writer builds GGUF files byte by byte (the layout llama.cpp writes: contiguous
header, tensor data at 32-byte aligned offsets relative to the data section).
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass

import numpy as np

from . import DType, UqError, Weights, _check, lib

ALIGN = 32

# value type ids (GgufValueType::from_id, gguf.rs:56-72)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_NUMPY = {U8: "<u1", I8: "<i1", U16: "<u2", I16: "<i2", U32: "<u4", I32: "<i4", F32: "<f4", BOOL: "<u1",
          U64: "<u8", I64: "<i8", F64: "<f8"}


class _Tensor(C.Structure):
    _fields_ = [("name", C.c_void_p), ("name_len", C.c_size_t), ("offset", C.c_uint64), ("nbytes", C.c_uint64),
                ("has_nbytes", C.c_int), ("ggml_type", C.c_uint32), ("n_dims", C.c_uint32),
                ("shape", C.POINTER(C.c_uint64)), ("n_elements", C.c_uint64)]


class _Kv(C.Structure):
    _fields_ = [("key", C.c_void_p), ("key_len", C.c_size_t), ("type", C.c_uint32), ("elem_type", C.c_uint32),
                ("count", C.c_uint64), ("data", C.c_void_p)]


@dataclass
class TensorMeta:
    """TensorMeta (unltd-model-loader/src/lib.rs:24-38); offset is absolute."""
    name: str
    offset: int
    nbytes: int | None
    dtype: str
    ggml_type_id: int
    shape: list
    n_elements: int


def type_blocksize(ggml_type: int):
    """ggml_type_blocksize (gguf.rs:193-234): (bytes, elements) or None."""
    b, e = C.c_uint64(), C.c_uint64()
    rc = lib().uq_gguf_type_blocksize(ggml_type, C.byref(b), C.byref(e))
    return (b.value, e.value) if rc == 0 else None


def type_name(ggml_type: int) -> str:
    """ggml_type_name (gguf.rs:237-278)."""
    buf = C.create_string_buffer(64)
    _check(lib().uq_gguf_type_name(ggml_type, buf, 64))
    return buf.value.decode()


class Gguf:
    """A validated GGUF file: header, metadata and tensor table; tensor bytes
    stay in the file's mapping until close()."""

    def __init__(self, h: C.c_void_p):
        self.h = h
        v, fs, ds, nkv, nt = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        _check(lib().uq_gguf_header(h, C.byref(v), C.byref(fs), C.byref(ds), C.byref(nkv), C.byref(nt)))
        self.version, self.file_size, self.data_start = v.value, fs.value, ds.value
        self._nkv, self._nt = nkv.value, nt.value
        self.metadata = [self._kv(i) for i in range(self._nkv)]
        self.tensors = [self._tensor(i) for i in range(self._nt)]

    @classmethod
    def open(cls, path) -> "Gguf":
        h = C.c_void_p()
        _check(lib().uq_gguf_open(str(path).encode(), C.byref(h)))
        return cls(h)

    @classmethod
    def parse(cls, data: bytes) -> "Gguf":
        b = np.frombuffer(bytes(data), np.uint8)
        h = C.c_void_p()
        _check(lib().uq_gguf_parse(b.ctypes.data_as(C.c_void_p) if b.size else None, b.size, C.byref(h)))
        return cls(h)

    def close(self):
        if self.h:
            _check(lib().uq_gguf_close(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # ------------------------------------------------------------ metadata
    def _kv(self, i: int):
        kv = _Kv()
        _check(lib().uq_gguf_kv_at(self.h, i, C.byref(kv)))
        key = C.string_at(kv.key, kv.key_len).decode("utf-8", "replace")
        if kv.elem_type == STRING:
            vals = [self._string(i, j) for j in range(kv.count)]
            return key, (vals[0] if kv.type == STRING else ("string", vals))
        a = np.frombuffer(C.string_at(kv.data, kv.count * np.dtype(_NUMPY[kv.elem_type]).itemsize),
                          _NUMPY[kv.elem_type]).copy()
        if kv.elem_type == BOOL:
            a = a != 0
        if kv.type == ARRAY:
            names = ["u8", "i8", "u16", "i16", "u32", "i32", "f32", "bool", "string", "array", "u64", "i64", "f64"]
            return key, (names[kv.elem_type], a.tolist())
        return key, a[0].item()

    def _string(self, i: int, j: int) -> str:
        p, n = C.c_void_p(), C.c_size_t()
        _check(lib().uq_gguf_kv_string(self.h, i, j, C.byref(p), C.byref(n)))
        return C.string_at(p, n.value).decode("utf-8", "replace")  # lossy, as String::from_utf8_lossy

    def get(self, key: str):
        """First value stored under key (gguf.rs:306-308), or None. Arrays
        come back as (element type name, list)."""
        for k, v in self.metadata:
            if k == key:
                return v
        return None

    def get_str(self, key: str):
        v = self.get(key)
        return v if isinstance(v, str) else None

    # -------------------------------------------------------------- tensors
    def _tensor(self, i: int) -> TensorMeta:
        t = _Tensor()
        _check(lib().uq_gguf_tensor_at(self.h, i, C.byref(t)))
        return TensorMeta(C.string_at(t.name, t.name_len).decode("utf-8", "replace"), t.offset,
                          t.nbytes if t.has_nbytes else None, type_name(t.ggml_type), t.ggml_type,
                          [t.shape[d] for d in range(t.n_dims)], t.n_elements)

    def find(self, name: str):
        """WeightIndex::find: the TensorMeta, or None when absent."""
        i = C.c_uint64()
        if lib().uq_gguf_find(self.h, name.encode(), C.byref(i)) != 0:
            return None
        return self.tensors[i.value]

    def tensor_bytes_summary(self):
        """(sum of known tensor bytes, number of tensors of unknown type)."""
        known = [t.nbytes for t in self.tensors if t.nbytes is not None]
        return sum(known), len(self.tensors) - len(known)

    def tensor(self, name: str):
        """MappedWeights::tensor: a copy of the tensor's bytes, or None when
        it is absent or of an unknown type."""
        p, n = C.c_void_p(), C.c_uint64()
        if lib().uq_gguf_tensor_bytes(self.h, name.encode(), C.byref(p), C.byref(n)) != 0:
            return None
        return np.frombuffer(C.string_at(p, n.value), np.uint8).copy()

    def tensor_checked(self, name: str, n_elements: int) -> np.ndarray:
        """MappedWeights::tensor_checked: raises UqError MISSING_TENSOR,
        ELEMENT_COUNT or GGML_TYPE."""
        p, n = C.c_void_p(), C.c_uint64()
        _check(lib().uq_gguf_tensor_checked(self.h, name.encode(), n_elements, C.byref(p), C.byref(n)))
        return np.frombuffer(C.string_at(p, n.value), np.uint8).copy()

    def check(self, name: str, n_elements: int, allowed) -> DType:
        """check (qwen35_forward.rs:109-128): the tensor's dtype."""
        mask = 0
        for d in allowed:
            mask |= 1 << int(d)
        d = C.c_int()
        _check(lib().uq_gguf_check(self.h, name.encode(), n_elements, mask, C.byref(d)))
        return DType(d.value)

    def upload(self, name: str) -> Weights:
        """The tensor's bytes, unchanged, in HBM: dim_in = shape[0]."""
        h = C.c_void_p()
        _check(lib().uq_gguf_upload(self.h, name.encode(), C.byref(h)))
        return Weights.from_handle(h)


class Writer:
    """Byte-level GGUF writer for fixtures (little-endian)."""

    def __init__(self):
        self.b = bytearray()

    def u32(self, v):
        self.b += struct.pack("<I", v)
        return self

    def u64(self, v):
        self.b += struct.pack("<Q", v)
        return self

    def raw(self, data: bytes):
        self.b += data
        return self

    def str(self, s):
        s = s.encode() if isinstance(s, str) else bytes(s)
        return self.u64(len(s)).raw(s)

    def pad_to(self, n: int):
        assert len(self.b) <= n, f"pad_to: already past {n}"
        self.b += bytes(n - len(self.b))
        return self

    def finish(self) -> bytes:
        return bytes(self.b)


def _value(w: Writer, vtype: int, v):
    if vtype == STRING:
        w.str(v)
    elif vtype == ARRAY:
        et, vals = v
        w.u32(et).u64(len(vals))
        for x in vals:
            _value(w, et, x)
    else:
        w.raw(np.array([v], _NUMPY[vtype]).tobytes())


def write(kvs, tensors, version: int = 3) -> bytes:
    """A whole GGUF file. kvs: [(key, value type, value)] (arrays as
    (element type, list)). tensors: [(name, shape, ggml type, bytes)], laid
    out in order at 32-byte aligned offsets of the data section."""
    w = Writer().raw(b"GGUF").u32(version).u64(len(tensors)).u64(len(kvs))
    for k, t, v in kvs:
        w.str(k).u32(t)
        _value(w, t, v)
    rel = 0
    offsets = []
    for name, shape, gt, data in tensors:
        offsets.append(rel)
        w.str(name).u32(len(shape))
        for d in shape:
            w.u64(d)
        w.u32(gt).u64(rel)
        rel = (rel + len(data) + ALIGN - 1) // ALIGN * ALIGN
    start = (len(w.b) + ALIGN - 1) // ALIGN * ALIGN
    w.pad_to(start)
    for (name, shape, gt, data), off in zip(tensors, offsets):
        w.pad_to(start + off).raw(bytes(data))
    return w.finish()
