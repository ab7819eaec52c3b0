"""CPU tests of the GGUF reader (engine_amd/csrc/gguf.cpp) through the C ABI.

- The reference's fixture file (crates/gguf/src/lib.rs:1219-1246) parses to
  the values its test asserts (lib.rs:1249-1276), and its invalid-magic and
  duplicate-metadata variants fail with those errors (lib.rs:1516-1546).
- Every other rule of the reader (lib.rs:185-272,1085-1199) is checked with a
  file built to break it: version, truncation, value types, bools, UTF-8,
  string/array/tensor limits, nesting depth, dimension count, alignment,
  offsets, tensor types and block geometry, missing tensors.
- Files from the independent writer (engine_amd/gguf_writer.py) round-trip: all
  metadata types, nested arrays, tensor directory and exact payload ranges.
Parsing needs no GPU.
"""
import struct

import numpy as np
import pytest

from engine_amd import gguf_writer as W


def E():
    import engine_amd
    return engine_amd


def reference_fixture() -> bytes:
    b = bytearray()
    b += struct.pack("<IIQQ", 0x46554747, 3, 1, 3)
    b += W.string("general.architecture") + struct.pack("<I", 8) + W.string("qwen3")
    b += W.string("general.alignment") + struct.pack("<II", 4, 32)
    b += W.string("test.array") + struct.pack("<IIQII", 9, 4, 2, 1, 0)
    b += W.string("token_embd.weight") + struct.pack("<IQQIQ", 2, 4, 8, 1, 0)
    b += b"\0" * 256
    return bytes(b)


def open_bytes(tmp_path, data: bytes, name="f.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return E().GgufFile.open(str(p))


def expect(tmp_path, data: bytes, kind: str):
    with pytest.raises(E().GgufError) as e:
        open_bytes(tmp_path, data)
    assert e.value.kind == kind, str(e.value)
    return e.value


def test_reference_fixture_parses_without_reading_tensor_data(tmp_path):
    g = open_bytes(tmp_path, reference_fixture())
    assert g.version() == 3
    assert g.tensor_count() == 1
    assert g.metadata("general.architecture") == "qwen3"
    assert g.metadata("general.alignment") == 32
    assert g.metadata("test.array") == [1, 0]
    t = g.tensors()[0]
    assert (t.name, t.dimensions, t.value_type, t.offset) == ("token_embd.weight", (4, 8), 1, 0)
    r = g.tensor_data_range("token_embd.weight")
    assert r.stop - r.start == 64
    assert r.start == g.tensor_data_offset()
    assert g.metadata("missing.key") is None
    assert list(g.metadata_map()) == sorted(["general.architecture", "general.alignment", "test.array"])


def test_reference_invalid_magic_and_duplicate_metadata(tmp_path):
    bad = bytearray(reference_fixture())
    bad[0] = 0
    err = expect(tmp_path, bytes(bad), "InvalidMagic")
    assert err.actual == 0x46554700
    dup = bytearray(reference_fixture())
    dup[16:24] = struct.pack("<Q", 4)
    entry = W.string("general.architecture") + struct.pack("<I", 8) + W.string("other")
    pos = bytes(dup).index(b"token_embd.weight") - 8
    dup[pos:pos] = entry
    err = expect(tmp_path, bytes(dup), "DuplicateMetadata")
    assert "general.architecture" in str(err)


def test_header_rules(tmp_path):
    expect(tmp_path, W.header(0, 0, version=2), "UnsupportedVersion")
    expect(tmp_path, W.header(0, 0)[:12], "Io")                       # truncated header
    expect(tmp_path, W.header(10_000_001, 0), "InvalidLength")        # tensor count limit
    expect(tmp_path, W.header(0, 1_000_001), "InvalidLength")         # metadata count limit
    expect(tmp_path, W.header(0, 1) + W.kv("a", 7, 1)[:-1] + b"\x02", "InvalidBool")
    expect(tmp_path, W.header(0, 1) + W.string("a") + struct.pack("<I", 13), "InvalidValueType")
    expect(tmp_path, W.header(0, 1) + W.string(b"\xff\xfe") + struct.pack("<I", 4) + b"\0" * 4, "InvalidUtf8")
    expect(tmp_path, W.header(0, 1) + struct.pack("<Q", 16 * 1024 * 1024 + 1), "InvalidLength")
    expect(tmp_path, W.header(0, 1) + W.string("a") + struct.pack("<IIQ", 9, 4, 1_000_001), "InvalidLength")
    # 17 nested arrays: depth 17 exceeds the limit of 16
    nest = W.string("a") + struct.pack("<I", 9) + struct.pack("<IQ", 9, 1) * 17 + struct.pack("<IQ", 4, 0)
    expect(tmp_path, W.header(0, 1) + nest, "ArrayNestingTooDeep")
    ok_nest = W.string("a") + struct.pack("<I", 9) + struct.pack("<IQ", 9, 1) * 15 + struct.pack("<IQI", 4, 1, 7)
    g = open_bytes(tmp_path, W.header(0, 1) + ok_nest + b"\0" * 32, "nest.gguf")
    v = g.metadata("a")
    for _ in range(16):
        assert isinstance(v, list) and len(v) == 1
        v = v[0]
    assert v == 7


def test_directory_rules(tmp_path):
    big = W.tensor_entry("t", [1] * 17, 0, 0)
    expect(tmp_path, W.header(1, 0) + big, "InvalidDimensionCount")
    # alignment must be a non-zero power of two
    expect(tmp_path, W.header(0, 1) + W.kv("general.alignment", W.U32, 24) + b"\0" * 64, "InvalidAlignment")
    expect(tmp_path, W.header(0, 1) + W.kv("general.alignment", W.U32, 0) + b"\0" * 64, "InvalidAlignment")
    # a signed alignment is not read as one (MetadataValue::as_u64): the default 32 applies
    g = open_bytes(tmp_path, W.header(0, 1) + W.kv("general.alignment", W.I32, 24) + b"\0" * 64, "signed.gguf")
    assert g.tensor_data_offset() % 32 == 0
    # tensor data offset past the end of the file
    expect(tmp_path, W.header(0, 0)[:24] + b"\0" * 3, "Truncated")
    # a tensor offset past the file
    data = W.header(1, 0) + W.tensor_entry("t", [4], 0, 4096)
    data += b"\0" * (32 - len(data) % 32)
    expect(tmp_path, data, "TensorOffsetOutOfBounds")


def test_tensor_range_rules(tmp_path):
    tensors = [("q4", [512, 2], 12, b"\1" * 576), ("bad_k", [300, 1], 12, b"\0" * 200),
               ("odd", [8], 5, b"\0" * 32), ("short", [256, 4], 12, b"\0" * 144)]
    g = open_bytes(tmp_path, W.build([("general.architecture", W.STRING, "x")], tensors))
    r = g.tensor_data_range("q4")
    assert r.stop - r.start == 576
    with pytest.raises(E().GgufError) as e:
        g.tensor_data_range("bad_k")
    assert e.value.kind == "QuantizationMismatch"
    with pytest.raises(E().GgufError) as e:
        g.tensor_data_range("odd")
    assert e.value.kind == "UnsupportedTensorType"
    with pytest.raises(E().GgufError) as e:
        g.tensor_data_range("short")   # 576 bytes declared, the file ends sooner
    assert e.value.kind == "TensorOffsetOutOfBounds"
    with pytest.raises(E().GgufError) as e:
        g.tensor_data_range("nope")
    assert e.value.kind == "MissingTensor"
    assert g.tensor("nope") is None


def test_writer_round_trip(tmp_path):
    rng = np.random.default_rng(1)
    md = [("general.architecture", W.STRING, "qwen3"), ("u8", W.U8, 250), ("i8", W.I8, -7), ("u16", W.U16, 65000),
          ("i16", W.I16, -30000), ("u32", W.U32, 4_000_000_000), ("i32", W.I32, -2_000_000_000),
          ("f32", W.F32, 1.5), ("b", W.BOOL, True), ("u64", W.U64, 2 ** 60), ("i64", W.I64, -(2 ** 60)),
          ("f64", W.F64, -2.25), ("s", W.STRING, "héllo"),
          ("strs", W.ARRAY, (W.STRING, ["a", "bc", ""])), ("fl", W.ARRAY, (W.F32, [0.5, -1.0]))]
    payloads = [("blk.0.w", [256, 3], 12, rng.integers(0, 256, 3 * 144, dtype=np.uint8).tobytes()),
                ("blk.0.n", [256], 0, W.f32_payload(rng.standard_normal(256))),
                ("blk.1.w", [512, 2], 14, rng.integers(0, 256, 2 * 2 * 210, dtype=np.uint8).tobytes())]
    for align in (32, 64):
        data = W.build(md, payloads, alignment=align)
        g = open_bytes(tmp_path, data, f"rt{align}.gguf")
        m = g.metadata_map()
        for k, _, v in md:
            got = m[k]
            want = list(v[1]) if isinstance(v, tuple) else v
            assert got == want, (k, got, want)
        assert list(m) == sorted(m)
        infos = g.tensors()
        assert [(t.name, list(t.dimensions), t.value_type) for t in infos] == [(n, d, t) for n, d, t, _ in payloads]
        for (name, _, _, payload) in payloads:
            r = g.tensor_data_range(name)
            assert data[r.start:r.stop] == payload
            assert r.start % align == 0


# Damaged files: every prefix of a well-formed file and seeded byte mutations
# of its header and directory. Each must open cleanly or fail with a
# GgufError; whatever opens is read back through every accessor. Run under
# ASan + UBSan by tests/test_sanitizers.py, these are the parser's memory-safety
# checks on untrusted input.

def _rich_file() -> bytes:
    rng = np.random.default_rng(7)
    md = [("general.architecture", W.STRING, "qwen3"), ("u8", W.U8, 250), ("i16", W.I16, -30000),
          ("u32", W.U32, 4_000_000_000), ("f32", W.F32, 1.5), ("b", W.BOOL, True), ("u64", W.U64, 2 ** 60),
          ("f64", W.F64, -2.25), ("s", W.STRING, "héllo"), ("strs", W.ARRAY, (W.STRING, ["a", "bc", ""])),
          ("nested", W.ARRAY, (W.ARRAY, [(W.I32, [1, -2]), (W.STRING, ["x"])])),
          ("fl", W.ARRAY, (W.F32, [0.5, -1.0]))]
    payloads = [("blk.0.w", [256, 3], 12, rng.integers(0, 256, 3 * 144, dtype=np.uint8).tobytes()),
                ("blk.0.n", [256], 0, W.f32_payload(rng.standard_normal(256))),
                ("blk.1.w", [512, 2], 14, rng.integers(0, 256, 2 * 2 * 210, dtype=np.uint8).tobytes())]
    return W.build(md, payloads, alignment=64)


def _read_all(g) -> None:
    g.version()
    g.tensor_data_offset()
    g.metadata_map()
    for t in g.tensors():
        try:
            g.tensor_data_range(t.name)
        except E().GgufError:
            pass
        g.tensor(t.name)
    g.close()


def _open_or_error(path, data: bytes):
    path.write_bytes(data)
    try:
        g = E().GgufFile.open(str(path))
    except E().GgufError as e:
        return e.kind
    _read_all(g)
    return None


def test_rich_file_opens_and_nested_arrays_read_back(tmp_path):
    data = _rich_file()
    g = open_bytes(tmp_path, data)
    assert g.metadata("nested") == [[1, -2], ["x"]]
    assert len(g.tensors()) == 3
    _read_all(g)


def test_every_truncation_fails_cleanly(tmp_path):
    data = _rich_file()
    g = open_bytes(tmp_path, data, "whole.gguf")
    data_start = g.tensor_data_offset()
    g.close()
    p = tmp_path / "cut.gguf"
    kinds = {}
    for n in range(len(data)):
        kind = _open_or_error(p, data[:n])
        if n < data_start:
            # header, metadata and directory are all required
            assert kind is not None, n
        kinds[kind] = kinds.get(kind, 0) + 1
    assert _open_or_error(p, data) is None
    assert {"Io", "Truncated"} & set(kinds), kinds


def test_mutated_headers_and_directories_fail_cleanly(tmp_path):
    data = _rich_file()
    g = open_bytes(tmp_path, data, "whole.gguf")
    data_start = g.tensor_data_offset()
    g.close()
    rng = np.random.default_rng(2024)
    p = tmp_path / "mut.gguf"
    failures = 0
    for i in range(1500):
        b = bytearray(data)
        if i % 3 == 0:
            # one 8-byte field overwritten with a large or boundary count
            pos = int(rng.integers(4, data_start - 8))
            v = [2 ** 64 - 1, 2 ** 63, 2 ** 32, 2 ** 32 - 1, 0x7FFF_FFFF, 17, 0][int(rng.integers(7))]
            b[pos:pos + 8] = struct.pack("<Q", v)
        else:
            for _ in range(int(rng.integers(1, 5))):
                b[int(rng.integers(4, data_start))] = int(rng.integers(0, 256))
        failures += _open_or_error(p, bytes(b)) is not None
    assert failures > 100  # the mutations reach the parser's checks
