"""GGUF reader through the C ABI (re_gguf_*), on the CPU: the reference's parser tests
(src/gguf.rs:1063-1312) on the same fixture bytes, the loader's tensor-byte range
(src/loader.rs:95-101) and the byte counts of quant.rs:75-101, plus the error paths the
reference's Reader reports (gguf.rs:212-312). Parsing and mapping touch no GPU."""
import struct

import numpy as np
import pytest

import ggufw as W
from rehip import Gguf, RehipError, RE_ERR_ARG, RE_ERR_SIZE, RE_ERR_TYPE


def _file(tmp_path, data: bytes, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return p


def _err(tmp_path, data: bytes) -> RehipError:
    with pytest.raises(RehipError) as e:
        Gguf(_file(tmp_path, data))
    return e.value


def test_parses_header_kv_and_tensor_info(tmp_path):
    b = W.synth_gguf()
    with Gguf(_file(tmp_path, b)) as f:
        assert (f.version, f.n_tensors, f.n_kv) == (3, 1, 3)
        assert f.data_offset == len(b)
        assert f.get("general.architecture") == "qwen2moe"
        assert f.get("general.block_count") == 48
        assert f.get("tokenizer.ggml.tokens") == ("Array", "Str", 2)
        assert f.get("absent.key") is None
        assert f.keys() == [("general.architecture", "Str"), ("general.block_count", "U32"),
                            ("tokenizer.ggml.tokens", "Array")]
        t = f.tensors[0]
        assert (t.name, t.dims, t.ggml_type, t.offset) == ("blk.0.ffn_gate_exps.weight", [2048, 512, 64], 12, 0)
        assert t.numel() == 2048 * 512 * 64


def test_alignment_defaults_when_absent(tmp_path):
    b = W.synth_gguf()
    with Gguf(_file(tmp_path, b)) as f:
        assert f.alignment() == 32
        assert f.data_start == (len(b) + 31) // 32 * 32


def test_header_only_file_has_no_tensor_bytes(tmp_path):
    # the fixture declares 2048*512*64 Q4_K elements but carries no data: the range check fails
    with Gguf(_file(tmp_path, W.synth_gguf())) as f:
        with pytest.raises(RehipError) as e:
            f.tensor_bytes("blk.0.ffn_gate_exps.weight")
        assert e.value.code == RE_ERR_SIZE and "out of bounds" in e.value.message


def test_rejects_bad_magic(tmp_path):
    b = bytearray(W.synth_gguf())
    b[0] = ord("X")
    e = _err(tmp_path, bytes(b))
    assert e.code == RE_ERR_ARG and e.message == "gguf parse error at 0: missing GGUF magic"


def test_rejects_truncated_buffer(tmp_path):
    full = W.synth_gguf()
    e = _err(tmp_path, full[: len(full) // 2])
    assert "unexpected EOF, need" in e.message
    for cut in (4, 6, 8, 20, 40, len(full) - 1):
        assert "gguf parse error at" in _err(tmp_path, full[:cut]).message


def test_rejects_unsupported_version(tmp_path):
    for v in (1, 4, 0xFFFFFFFF):
        b = bytearray(W.synth_gguf())
        b[4:8] = struct.pack("<I", v)
        e = _err(tmp_path, bytes(b))
        assert e.message == f"gguf parse error at 4: unsupported GGUF version {v} (need 2 or 3)"


def test_version2_uses_u32_counts(tmp_path):
    b = W.header([("a.b", W.U32, 7)], [("t", [32], 0, 0)], version=2)
    with Gguf(_file(tmp_path, b + bytes(256))) as f:
        assert (f.version, f.n_tensors, f.n_kv) == (2, 1, 1)
        assert f.get("a.b") == 7
        assert f.data_offset == len(b)
        assert f.tensor_bytes("t").size == 128


def test_every_value_kind(tmp_path):
    kvs = [("u8", W.U8, 255), ("i8", W.I8, -128), ("u16", W.U16, 65535), ("i16", W.I16, -32768),
           ("u32", W.U32, 4294967295), ("i32", W.I32, -2147483648), ("f32", W.F32, 1.5), ("bool", W.BOOL, True),
           ("str", W.STR, "héllo"), ("empty", W.STR, ""), ("u64", W.U64, 2**64 - 1), ("i64", W.I64, -2**63),
           ("f64", W.F64, -2.25), ("arr", W.ARRAY, (W.ARRAY, [(W.U8, [1, 2]), (W.STR, ["x"])])),
           ("u8", W.U32, 9)]   # a repeated key: the first one wins (gguf.rs:139-141)
    with Gguf(_file(tmp_path, W.header(kvs, []))) as f:
        assert f.n_kv == len(kvs)
        got = {k: f.get(k) for k, _, _ in kvs}
        assert got["u8"] == 255 and got["i8"] == -128 and got["u16"] == 65535 and got["i16"] == -32768
        assert got["u32"] == 4294967295 and got["i32"] == -2147483648
        assert got["f32"] == 1.5 and got["bool"] is True and got["str"] == "héllo" and got["empty"] == ""
        assert got["u64"] == -1   # U64 reads back through int64 (two's complement)
        assert got["i64"] == -2**63 and got["f64"] == -2.25
        assert got["arr"] == ("Array", "Array", 2)


def test_value_errors_name_offset_and_key(tmp_path):
    b = W.header([("ok", W.U8, 1)], [])
    bad = b[:-1 - 4] + struct.pack("<I", 13) + b[-1:]   # kind 13 for key "ok"
    e = _err(tmp_path, bad)
    assert e.message == f"gguf parse error at {len(b) - 1}: unknown value kind 13 for key ok"
    # array element kind out of range
    b = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + W.gstr("a") + struct.pack("<II", W.ARRAY, 99) + bytes(16)
    assert "unknown array element kind 99" in _err(tmp_path, b).message
    # array count larger than the bytes left
    b = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + W.gstr("a") + struct.pack("<IIQ", W.ARRAY, W.U8, 100) + bytes(10)
    e = _err(tmp_path, b)
    assert e.message == f"gguf parse error at {len(b) - 10}: array count 100 exceeds remaining bytes"


def test_rejects_more_than_8_dims(tmp_path):
    b = W.header([], [("t9", [1] * 9, 0, 0)])
    pos = b.index(struct.pack("<I", 9), 24 + 10) + 4
    e = _err(tmp_path, b)
    assert e.message == f"gguf parse error at {pos}: tensor t9 declares 9 dims (max 8)"


def test_rejects_invalid_utf8(tmp_path):
    for raw, tail in ((b"a\xffb", "invalid utf-8 sequence of 1 bytes from index 1"),
                      (b"ab\xe2\x82", "incomplete utf-8 byte sequence from index 2"),
                      (b"\xe2\x28\xa1", "invalid utf-8 sequence of 1 bytes from index 0"),
                      (b"x\xf0\x9f\x98(", "invalid utf-8 sequence of 3 bytes from index 1"),
                      (b"\xed\xa0\x80", "invalid utf-8 sequence of 1 bytes from index 0")):
        b = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + W.gstr(raw) + struct.pack("<IB", W.U8, 1)
        e = _err(tmp_path, b)
        assert e.message == f"gguf parse error at 32: invalid utf-8 string: {tail}", raw


def test_tensor_entry_numel_and_nbytes_math(tmp_path):
    rng = np.random.default_rng(0)
    cases = [("f32", [128], 0, 512), ("f16", [6], 1, 12), ("bf16", [4], 30, 8), ("q40", [256], 2, 144),
             ("q50", [64], 6, 44), ("q80", [32, 2], 8, 68), ("q4k", [256], 12, 144), ("q5k", [512], 13, 352),
             ("mat", [896, 4864], 14, 896 * 4864 // 256 * 210)]
    data = [rng.integers(0, 256, nb, dtype=np.uint8).tobytes() for *_, nb in cases]
    tensors = [(n, d, t, x) for (n, d, t, _), x in zip(cases, data)]
    with Gguf(_file(tmp_path, W.write([], tensors))) as f:
        for (name, _, _, nb), x in zip(cases, data):
            got = f.tensor_bytes(name)
            assert got.size == nb and got.tobytes() == x, name
            assert not got.flags.writeable


def test_unsized_types_and_partial_blocks(tmp_path):
    tensors = [("q4k_partial", [100], 12, bytes(144)), ("i8", [16], 24, bytes(16)), ("iq2", [256], 16, bytes(66))]
    with Gguf(_file(tmp_path, W.write([], tensors))) as f:
        for name, *_ in tensors:
            with pytest.raises(RehipError) as e:
                f.tensor_bytes(name)
            assert e.value.code == RE_ERR_TYPE, name


def test_writer_round_trip_raw_bytes_and_alignment(tmp_path):
    raw = bytes(144)
    f32 = np.array([0.5, -0.5], np.float32).tobytes()
    b = W.write([("general.alignment", W.U32, 64), ("general.architecture", W.STR, "test")],
                [("t0", [256], 12, raw), ("t1", [2], 0, f32)], alignment=64)
    with Gguf(_file(tmp_path, b)) as f:
        assert f.alignment() == 64 and len(f.tensors) == 2
        assert f.data_start % 64 == 0 and f.data_start == (f.data_offset + 63) // 64 * 64
        assert all(t.offset % 64 == 0 for t in f.tensors)
        assert f.tensor_bytes("t0").tobytes() == raw
        assert np.frombuffer(f.tensor_bytes("t1").tobytes(), np.float32).tolist() == [0.5, -0.5]


def test_u64_alignment_and_out_of_range_offset(tmp_path):
    hdr = W.header([("general.alignment", W.U64, 128)], [("in", [32], 0, 0), ("past", [32], 0, 4096)])
    start = (len(hdr) + 127) // 128 * 128
    b = hdr + bytes(start - len(hdr)) + bytes(128)
    with Gguf(_file(tmp_path, b)) as f:
        assert f.alignment() == 128 and f.data_start == start
        assert f.tensor_bytes("in").size == 128
        with pytest.raises(RehipError) as e:
            f.tensor_bytes("past")
        assert e.value.code == RE_ERR_SIZE


def test_duplicate_tensor_names_resolve_to_the_first(tmp_path):
    b = W.write([], [("w", [32], 0, np.ones(32, np.float32).tobytes()),
                     ("w", [32], 0, np.zeros(32, np.float32).tobytes())])
    with Gguf(_file(tmp_path, b)) as f:
        assert np.frombuffer(f.tensor_bytes("w").tobytes(), np.float32).sum() == 32


def test_missing_and_empty_files(tmp_path):
    with pytest.raises(RehipError):
        Gguf(tmp_path / "absent.gguf")
    with pytest.raises(RehipError):
        Gguf(_file(tmp_path, b""))
    with pytest.raises(RehipError) as e:
        Gguf(_file(tmp_path, b"GGU"))
    assert "missing GGUF magic" in e.value.message
