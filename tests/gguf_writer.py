"""A small, independent GGUF writer and reader for the tests (the format of the GGUF spec, as the reference reads it
in crates/inference-tensor/src/quantized/gguf_file.rs).  Values are (type_id, python value) pairs so every one of
the 13 value types can be written exactly; arrays are (9, (elem_type_id, [python values])).  The tests write
files with it and check the library's C++ reader against what went in, and read the C++ writer's files back."""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
        F64: "<d"}


def _len(n, version):
    return struct.pack("<I" if version == 1 else "<Q", n)


def _string(s, version):
    b = s.encode() if isinstance(s, str) else s
    return _len(len(b), version) + b


def value_bytes(t, v, version=3):
    if t in _FMT:
        return struct.pack(_FMT[t], int(v) if t == BOOL else v)
    if t == STRING:
        return _string(v, version)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<I", et) + _len(len(items), version)
        if et in _FMT:  # fixed-size elements in one pack
            return out + struct.pack("<%d%s" % (len(items), _FMT[et][1]), *[int(x) if et == BOOL else x for x in items])
        return out + b"".join(value_bytes(et, it, version) for it in items)
    raise ValueError(t)


def kv_bytes(metadata, version=3):
    """metadata: [(key, type_id, value)] -> the serialized key/value entries."""
    out = b""
    for key, t, v in metadata:
        out += _string(key, version) + struct.pack("<I", t) + value_bytes(t, v, version)
    return out


def write(path, metadata, tensors, version=3, alignment=32, magic=0x46554747, raw_kv=None):
    """tensors: [(name, dims outermost first, ggml type id, bytes)].  Tensor data is aligned to `alignment` (the
    caller puts general.alignment in metadata when it is not 32)."""
    kv = raw_kv if raw_kv is not None else kv_bytes(metadata, version)
    head = struct.pack("<II", magic, version) + _len(len(tensors), version) + _len(len(metadata), version) + kv
    offset = 0
    table = b""
    offsets = []
    for name, dims, dtype, data in tensors:
        table += _string(name, version) + struct.pack("<I", len(dims))
        for d in reversed(dims):
            table += struct.pack("<I" if version == 1 else "<Q", d)
        table += struct.pack("<IQ", dtype, offset)
        offsets.append(offset)
        offset += len(data)
        offset = (offset + alignment - 1) // alignment * alignment
    pos = len(head) + len(table)
    data_start = (pos + alignment - 1) // alignment * alignment
    body = bytearray(head + table + b"\0" * (data_start - pos))
    for (name, dims, dtype, data), off in zip(tensors, offsets):
        body += b"\0" * (data_start + off - len(body))
        body += data
    with open(path, "wb") as f:
        f.write(bytes(body))
    return data_start, offsets


def read(path):
    """A minimal reader of version 2/3 files: (version, {key: (type, value)}, [(name, dims, type, offset)],
    data_start)."""
    with open(path, "rb") as f:
        b = f.read()
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, b, pos)
        pos += struct.calcsize(fmt)
        return v[0]

    def string():
        nonlocal pos
        n = take("<Q")
        s = b[pos:pos + n]
        pos += n
        return s.decode()

    def value(t):
        if t in _FMT:
            v = take(_FMT[t])
            return bool(v) if t == BOOL else v
        if t == STRING:
            return string()
        et = take("<I")
        n = take("<Q")
        return (et, [value(et) for _ in range(n)])

    magic, version = take("<I"), take("<I")
    assert magic == 0x46554747 and version in (2, 3), (magic, version)
    nt, nkv = take("<Q"), take("<Q")
    meta = {}
    for _ in range(nkv):
        k = string()
        t = take("<I")
        meta[k] = (t, value(t))
    tensors = []
    for _ in range(nt):
        name = string()
        nd = take("<I")
        dims = [take("<Q") for _ in range(nd)][::-1]
        tensors.append((name, dims, take("<I"), take("<Q")))
    align = meta.get("general.alignment", (U32, 32))[1]
    return version, meta, tensors, (pos + align - 1) // align * align
