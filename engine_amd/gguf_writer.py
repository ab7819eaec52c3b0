"""A small GGUF v3 writer (written from the published GGUF format:
little-endian header "GGUF", version, tensor count, metadata count, typed
key/value entries, the tensor directory, then tensor data at the aligned end
of the directory, each tensor at its own aligned offset)."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", U64: "<Q", I64: "<q",
        F64: "<d"}


def string(s) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(vtype: int, v) -> bytes:
    if vtype in _FMT:
        return struct.pack(_FMT[vtype], v)
    if vtype == BOOL:
        return struct.pack("<B", 1 if v else 0)
    if vtype == STRING:
        return string(v)
    if vtype == ARRAY:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(value(etype, x) for x in items)
    raise ValueError(vtype)


def header(tensor_count: int, metadata_count: int, version: int = 3, magic: int = 0x46554747) -> bytes:
    return struct.pack("<IIQQ", magic, version, tensor_count, metadata_count)


def kv(key: str, vtype: int, v) -> bytes:
    return string(key) + struct.pack("<I", vtype) + value(vtype, v)


def tensor_entry(name: str, dims, vtype: int, offset: int) -> bytes:
    return string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", vtype, offset)


def build(metadata, tensors, alignment: int = 32, extra_tail: int = 0) -> bytes:
    """metadata: [(key, type, value)]; tensors: [(name, dims, type, payload bytes)].
    general.alignment is written when it differs from 32."""
    md = list(metadata)
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in md):
        md.append(("general.alignment", U32, alignment))
    offsets, pos = [], 0
    for _, _, _, payload in tensors:
        pos = (pos + alignment - 1) // alignment * alignment
        offsets.append(pos)
        pos += len(payload)
    out = bytearray(header(len(tensors), len(md)))
    for k, t, v in md:
        out += kv(k, t, v)
    for (name, dims, vtype, _), off in zip(tensors, offsets):
        out += tensor_entry(name, dims, vtype, off)
    data_start = (len(out) + alignment - 1) // alignment * alignment
    out += b"\0" * (data_start - len(out))
    for (_, _, _, payload), off in zip(tensors, offsets):
        out += b"\0" * (data_start + off - len(out))
        out += bytes(payload)
    out += b"\0" * extra_tail
    return bytes(out)


def f32_payload(a) -> bytes:
    return np.ascontiguousarray(a, np.float32).tobytes()


def write(path, metadata, tensors, alignment: int = 32) -> int:
    """Streams a GGUF file to `path` without building it in memory: tensors are
    (name, dims, type, payload) with payload bytes or a numpy array. Returns
    the file size."""
    md = list(metadata)
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in md):
        md.append(("general.alignment", U32, alignment))
    sizes = [memoryview(p).nbytes if not isinstance(p, np.ndarray) else p.nbytes for _, _, _, p in tensors]
    offsets, pos = [], 0
    for n in sizes:
        pos = (pos + alignment - 1) // alignment * alignment
        offsets.append(pos)
        pos += n
    head = bytearray(header(len(tensors), len(md)))
    for k, t, v in md:
        head += kv(k, t, v)
    for (name, dims, vtype, _), off in zip(tensors, offsets):
        head += tensor_entry(name, dims, vtype, off)
    data_start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_start - len(head)))
        written = 0
        for (_, _, _, payload), off, n in zip(tensors, offsets, sizes):
            f.write(b"\0" * (off - written))
            f.write(payload.tobytes() if isinstance(payload, np.ndarray) else payload)
            written = off + n
        return f.tell()

