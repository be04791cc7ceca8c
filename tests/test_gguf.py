"""GGUF reader (include/uq_gguf.h) against the reference loader's own tests.

Each test below restates one of crates/unltd-model-loader/src/gguf.rs's
tests (:763-1089) or weights.rs's (:98-183) with the same fixture bytes and
the same expected values; the refusals are checked by status code (the
reference's LoadError variant) and by the offsets the reference asserts.
The reader needs no GPU: these run on the CPU.
"""
import os
import re

import numpy as np
import pytest

import uq
from uq import DType
from uq import gguf as G
from uq.gguf import Writer as W


def parse(b):
    return G.Gguf.parse(b)


def refused(kind, b):
    with pytest.raises(uq.UqError) as e:
        parse(b)
    assert e.value.kind == kind, str(e.value)
    return str(e.value)


def fixture_valid():
    """gguf.rs:809-848: v3, 2 kv, 2 tensors (F32 [4,3] at rel 0, Q8_0 [33] at
    rel 64); data_start 224, file padded to 356. (The infos end at byte 214;
    the reference's comment says 217, which rounds up to the same 224.)"""
    h = (W().raw(b"GGUF").u32(3).u64(2).u64(2)
         .str("general.architecture").u32(8).str("llama")
         .str("test.counts").u32(9).u32(4).u64(3).u32(10).u32(20).u32(30)
         .str("tok_embd.weight").u32(2).u64(4).u64(3).u32(0).u64(0)
         .str("norm.weight").u32(1).u64(33).u32(8).u64(64))
    data_start = (len(h.b) + 31) // 32 * 32
    assert data_start == 224
    return h.pad_to(data_start + 64 + 68).finish()


def test_parses_valid_v3():  # gguf.rs:850-884
    b = fixture_valid()
    g = parse(b)
    assert g.version == 3 and g.file_size == len(b) and g.data_start == 224
    assert len(g.metadata) == 2
    assert g.get_str("general.architecture") == "llama"
    assert g.get("test.counts") == ("u32", [10, 20, 30])
    assert len(g.tensors) == 2
    t0, t1 = g.tensors
    assert (t0.name, t0.shape, t0.n_elements, t0.nbytes, t0.dtype, t0.offset) == \
        ("tok_embd.weight", [4, 3], 12, 48, "F32", 224)
    assert (t1.shape, t1.nbytes, t1.dtype, t1.offset) == ([33], 68, "Q8_0", 288)
    assert len(g.tensors) == 2
    assert g.find("tok_embd.weight") is not None
    assert g.find("ausente") is None


def test_rejects_bad_magic():  # gguf.rs:886-893
    msg = refused("MAGIC", W().raw(b"NOPE").u32(3).u64(0).u64(0).finish())
    assert "4E, 4F, 50, 45" in msg  # the magic read back


@pytest.mark.parametrize("v", [1, 4])
def test_rejects_unsupported_version(v):  # gguf.rs:895-904
    msg = refused("VERSION", W().raw(b"GGUF").u32(v).u64(0).u64(0).finish())
    assert f"version {v}" in msg


def test_rejects_implausible_counts():  # gguf.rs:906-914
    refused("FILE", W().raw(b"GGUF").u32(3).u64(0).u64(1 << 40).finish())
    refused("FILE", W().raw(b"GGUF").u32(3).u64(1 << 40).u64(0).finish())


def test_rejects_truncated_file():  # gguf.rs:916-922
    full = fixture_valid()
    refused("FILE", full[: len(full) // 2])


def test_rejects_huge_string_len():  # gguf.rs:924-935
    refused("FILE", W().raw(b"GGUF").u32(3).u64(0).u64(1).u64(1 << 50).finish())


def header_one_tensor(name, n_dims, dims, ggml_type, raw_offset):  # gguf.rs:940-958
    w = W().raw(b"GGUF").u32(3).u64(1).u64(0).str(name).u32(n_dims)
    for d in dims:
        w.u64(d)
    return w.u32(ggml_type).u64(raw_offset).finish()


def test_rejects_zero_dims_and_zero_elements():  # gguf.rs:960-984
    refused("FILE", W().raw(b"GGUF").u32(3).u64(1).u64(0).str("w").u32(0).finish())
    refused("FILE", W().raw(b"GGUF").u32(3).u64(1).u64(0).str("w").u32(1).u64(0).u32(0).u64(0).finish())


def test_rejects_tensor_out_of_bounds():  # gguf.rs:986-1004
    msg = refused("TENSOR_BOUNDS", header_one_tensor("w", 1, [4], 0, 0))
    assert re.search(r"tensor 'w' claims bytes \[64, 64\+16\) beyond file size 57", msg), msg


def test_rejects_misaligned_tensor():  # gguf.rs:1006-1021
    msg = refused("TENSOR_ALIGN", header_one_tensor("w", 1, [4], 0, 100))
    assert "tensor 'w' at offset 164 is not aligned to 32 bytes" in msg


def test_rejects_overlapping_tensors():  # gguf.rs:1023-1054
    b = (W().raw(b"GGUF").u32(3).u64(2).u64(0)
         .str("a").u32(1).u64(4).u32(0).u64(0)
         .str("b").u32(1).u64(4).u32(0).u64(0)
         .pad_to(128).finish())
    msg = refused("TENSOR_OVERLAP", b)
    assert "'a' ends at 112, 'b' starts at 96" in msg


def test_tolerates_unknown_type_without_guessing():  # gguf.rs:1056-1065
    g = parse(header_one_tensor("w", 1, [4], 999, 0))
    assert g.tensors[0].nbytes is None
    assert g.tensors[0].dtype == "unknown(999)"
    assert g.tensor_bytes_summary() == (0, 1)
    assert sum(t.nbytes is None for t in g.tensors) == 1


def test_rejects_unknown_value_type():  # gguf.rs:1067-1077
    refused("FILE", W().raw(b"GGUF").u32(3).u64(0).u64(1).str("k").u32(77).finish())


def test_table_sizes_match_llama_cpp():  # gguf.rs:1079-1089
    assert G.type_blocksize(0) == (4, 1)
    assert G.type_blocksize(1) == (2, 1)
    assert G.type_blocksize(30) == (2, 1)
    assert G.type_blocksize(8) == (34, 32)
    assert G.type_blocksize(12) == (144, 256)
    assert G.type_blocksize(14) == (210, 256)
    assert G.type_blocksize(15) == (292, 256)
    assert G.type_blocksize(31) is None
    assert G.type_blocksize(34) == (54, 256)
    assert G.type_blocksize(999) is None


def test_block_sizes_agree_with_the_quant_kernels():
    """The loader's table and the kernels' block geometry are one fact."""
    for dt, (bb, be) in ((DType.Q4K, (144, 256)), (DType.Q6K, (210, 256)), (DType.Q8_0, (34, 32)),
                         (DType.F32, (4, 1))):
        assert G.type_blocksize(int(dt)) == (bb, be)
        assert uq.row_bytes(dt, 4096) == 4096 // be * bb


# -------------------------------------------------------------- weights.rs

@pytest.fixture
def tmp_gguf(tmp_path):
    def make(b):
        p = tmp_path / f"f{len(list(tmp_path.iterdir()))}.gguf"
        p.write_bytes(b)
        return p
    return make


def test_tensor_slices_are_the_file_bytes(tmp_gguf):  # weights.rs:124-143
    b = bytearray(fixture_valid())
    b[224], b[230], b[300] = 0xAB, 0xCD, 0xEF
    with G.Gguf.open(tmp_gguf(bytes(b))) as mw:
        assert mw.file_size == len(b)
        t0 = mw.tensor("tok_embd.weight")
        assert len(t0) == 48 and t0[0] == 0xAB and t0[6] == 0xCD
        t1 = mw.tensor("norm.weight")
        assert len(t1) == 68 and t1[12] == 0xEF


def test_tensor_none_for_absent(tmp_gguf):  # weights.rs:145-150
    with G.Gguf.open(tmp_gguf(fixture_valid())) as mw:
        assert mw.tensor("no.existe") is None


def test_tensor_checked_refusals(tmp_gguf):  # weights.rs:152-175
    with G.Gguf.open(tmp_gguf(fixture_valid())) as mw:
        assert len(mw.tensor_checked("tok_embd.weight", 12)) == 48
        with pytest.raises(uq.UqError) as e:
            mw.tensor_checked("tok_embd.weight", 13)
        assert e.value.kind == "ELEMENT_COUNT" and "has 12 elements, expected 13" in str(e.value)
        with pytest.raises(uq.UqError) as e:
            mw.tensor_checked("no.existe", 1)
        assert e.value.kind == "MISSING_TENSOR" and "no.existe" in str(e.value)


def test_open_refuses_truncated_file(tmp_gguf):  # weights.rs:177-182
    b = fixture_valid()
    with pytest.raises(uq.UqError):
        G.Gguf.open(tmp_gguf(b[:-40]))


def test_open_missing_file_is_io(tmp_path):
    with pytest.raises(uq.UqError) as e:
        G.Gguf.open(tmp_path / "absent.gguf")
    assert e.value.kind == "IO"


# ------------------------------------------- beyond the reference's own tests

def test_every_prefix_of_a_valid_file_is_refused_cleanly():
    """A file cut anywhere is refused (never a crash, never a partial read):
    short reads are BadFile, and once the header is whole the tensors run
    past the end (TensorOutOfBounds)."""
    b = fixture_valid()
    infos_end = 214  # magic..counts 24, two pairs 92, two tensor infos 98
    for n in range(len(b)):
        with pytest.raises(uq.UqError) as e:
            parse(b[:n])
        assert e.value.kind == ("FILE" if n < infos_end else "TENSOR_BOUNDS"), (n, str(e.value))
    parse(b)


def test_random_byte_corruptions_never_crash():
    rng = np.random.default_rng(7)
    b = np.frombuffer(fixture_valid(), np.uint8)
    for _ in range(2000):
        c = b.copy()
        idx = rng.integers(0, len(c), rng.integers(1, 4))
        c[idx] = rng.integers(0, 256, idx.size)
        try:
            g = parse(c.tobytes())
        except uq.UqError as e:
            assert e.kind in uq.STATUS.values()
            continue
        for t in g.tensors:  # what parses is in range
            if t.nbytes is not None:
                assert t.offset % 32 == 0 and t.offset + t.nbytes <= g.file_size


def test_metadata_value_types_round_trip():
    kvs = [("a.u8", G.U8, 200), ("a.i8", G.I8, -5), ("a.u16", G.U16, 65000), ("a.i16", G.I16, -300),
           ("a.u32", G.U32, 4000000000), ("a.i32", G.I32, -7), ("a.f32", G.F32, 1.5), ("a.bool", G.BOOL, True),
           ("a.str", G.STRING, "héllo"), ("a.u64", G.U64, 1 << 40), ("a.i64", G.I64, -(1 << 40)),
           ("a.f64", G.F64, 0.1), ("a.arr", G.ARRAY, (G.STRING, ["x", "", "yz"])),
           ("a.arr2", G.ARRAY, (G.F32, [1.0, -2.0])), ("a.u8", G.U8, 1)]
    g = parse(G.write(kvs, []))
    got = dict(reversed(g.metadata))  # first occurrence wins, as get()
    assert got["a.u8"] == 200 and g.get("a.u8") == 200
    assert got["a.i8"] == -5 and got["a.u16"] == 65000 and got["a.i16"] == -300
    assert got["a.u32"] == 4000000000 and got["a.i32"] == -7 and got["a.f32"] == 1.5
    assert got["a.bool"] is True and got["a.str"] == "héllo"
    assert got["a.u64"] == 1 << 40 and got["a.i64"] == -(1 << 40) and got["a.f64"] == 0.1
    assert got["a.arr"] == ("string", ["x", "", "yz"]) and got["a.arr2"] == ("f32", [1.0, -2.0])
    assert g.data_start % 32 == 0 and not g.tensors


def test_nested_array_and_alignment_refusals():
    nested = W().raw(b"GGUF").u32(3).u64(0).u64(1).str("k").u32(9).u32(9).u64(0).pad_to(64).finish()
    assert "nested array" in refused("FILE", nested)
    refused("FILE", G.write([("general.alignment", G.U32, 64)], []))
    parse(G.write([("general.alignment", G.U32, 32)], []))
    parse(G.write([("general.alignment", G.U64, 64)], []))  # only a u32 is read, as the reference


def test_repeated_tensor_name_finds_the_last():
    b = G.write([], [("w", [4], 0, bytes(16)), ("w", [8], 0, bytes(32))])
    g = parse(b)
    assert g.find("w").shape == [8]


def test_check_mirrors_qwen35_open():  # qwen35_forward.rs:109-128
    q4 = bytes(144 * 2)
    b = G.write([], [("blk.0.ffn_up.weight", [256, 2], 12, q4), ("blk.0.attn_norm.weight", [256], 0, bytes(1024)),
                     ("odd", [4], 2, bytes(18))])
    g = parse(b)
    assert g.check("blk.0.ffn_up.weight", 512, [DType.Q4K]) == DType.Q4K
    assert g.check("blk.0.ffn_up.weight", 512, [DType.Q4K, DType.Q6K]) == DType.Q4K
    assert g.check("blk.0.attn_norm.weight", 256, [DType.F32]) == DType.F32
    for args, kind in ((("missing", 1, [DType.F32]), "MISSING_TENSOR"),
                       (("blk.0.ffn_up.weight", 511, [DType.Q4K]), "ELEMENT_COUNT"),
                       (("blk.0.ffn_up.weight", 512, [DType.Q6K]), "FILE"),
                       (("odd", 4, [DType.F32]), "GGML_TYPE")):  # Q4_0 has no engine dtype
        with pytest.raises(uq.UqError) as e:
            g.check(*args)
        assert e.value.kind == kind, (args, str(e.value))


def test_upload_needs_a_device_and_fails_loudly_without_one():
    if uq.device_count() > 0:
        pytest.skip("a device is present")
    g = parse(G.write([], [("w", [256, 2], 12, bytes(288))]))
    with pytest.raises(uq.UqError) as e:
        g.upload("w")
    assert e.value.kind == "NO_DEVICE"
    with pytest.raises(uq.UqError) as e:
        g.upload("absent")
    assert e.value.kind == "MISSING_TENSOR"
