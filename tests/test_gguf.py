"""CPU tests of the GGUF reader / writer of the host layer (host/gguf.cpp; the reference's gguf_file.rs).

Files are written by an independent Python writer (tests/gguf_writer.py) and read through the C API, so every value
type, the three versions, alignment, the tensor table's dimension order, tensor bytes and each rejection of a
malformed file are checked against what went in; the C++ writer's output is read back by the Python reader.  The
two unit tests in gguf_file.rs (summary skips long arrays; long fixed-size arrays are located, not parsed) are
restated with the same shapes."""
import ctypes
import struct

import numpy as np
import pytest

import gguf_writer as G
import oracle as O
import qmm

ALL_VALUES = [
    ("general.architecture", G.STRING, "llama"),
    ("v.u8", G.U8, 200), ("v.i8", G.I8, -100), ("v.u16", G.U16, 60000), ("v.i16", G.I16, -30000),
    ("v.u32", G.U32, 4000000000), ("v.i32", G.I32, -2000000000), ("v.u64", G.U64, 2 ** 63 + 5),
    ("v.i64", G.I64, -2 ** 62), ("v.f32", G.F32, 0.1), ("v.f64", G.F64, -1e300), ("v.true", G.BOOL, True),
    ("v.false", G.BOOL, False), ("v.nul_padded", G.STRING, "name\0\0"), ("v.utf8", G.STRING, "héllo"),
    ("v.arr_u32", G.ARRAY, (G.U32, [1, 2, 3])), ("v.arr_str", G.ARRAY, (G.STRING, ["a", "bc"])),
    ("v.nested", G.ARRAY, (G.ARRAY, [(G.I8, [1, -1]), (G.I8, [])])), ("v.empty", G.ARRAY, (G.F32, [])),
]


def qbytes(gtype, n, k, seed):
    rng = np.random.default_rng(seed)
    return O.quantize(gtype, (rng.standard_normal((n, k)) * 0.02).astype(np.float32)).reshape(-1).tobytes()


def sample_tensors():
    f32 = np.arange(24, dtype=np.float32).tobytes()
    return [
        ("blk.0.attn_q.weight", [8, 256], O.Q4K, qbytes(O.Q4K, 8, 256, 1)),
        ("blk.0.ffn_down.weight", [4, 512], O.Q6K, qbytes(O.Q6K, 4, 512, 2)),
        ("token_embd.weight", [3, 64], O.Q8_0, qbytes(O.Q8_0, 3, 64, 3)),
        ("output_norm.weight", [24], 0, f32),
        ("expert.weight", [2, 3, 256], O.Q4K, qbytes(O.Q4K, 6, 256, 4)),
    ]


def open_file(path, summary=False):
    return qmm.GgufFile(str(path), summary)


@pytest.mark.parametrize("version", [1, 2, 3])
def test_reads_every_value_type_and_the_tensor_table(tmp_path, version):
    p = tmp_path / f"v{version}.gguf"
    tensors = sample_tensors()
    data_start, offsets = G.write(p, ALL_VALUES, tensors, version=version)
    with open_file(p) as g:
        assert g.version == version
        assert g.tensor_data_offset == data_start
        assert sorted(g.keys()) == sorted(k for k, _, _ in ALL_VALUES)
        for key, t, v in ALL_VALUES:
            assert g.value_type(key) == t, key
            if t in (G.U8, G.U16, G.U32, G.U64):
                assert g.u64(key) == v
            elif t in (G.I8, G.I16, G.I32, G.I64):
                assert g.i64(key) == v
            elif t == G.F32:
                assert g.f64(key) == struct.unpack("<f", struct.pack("<f", v))[0]
            elif t == G.F64:
                assert g.f64(key) == v
            elif t == G.BOOL:
                assert g.u64(key) == int(v)  # Value::to_u64 upcasts bool
            elif t == G.STRING:
                assert g.string(key) == v.rstrip("\0")  # trailing NULs are dropped (gguf_file.rs:160-163)
            else:
                n, et = g.array(key)
                assert n == len(v[1]) and (et == v[0] if n else et == -1)
        got = g.tensors()
        assert got == [(n, t, d, o) for (n, d, t, _), o in zip(tensors, offsets)]


def test_accessors_check_their_type(tmp_path):
    p = tmp_path / "a.gguf"
    G.write(p, ALL_VALUES, [])
    with open_file(p) as g:
        with pytest.raises(qmm.QmmError, match="not a"):
            g.u64("v.i8")  # to_u64 does not take signed values
        with pytest.raises(qmm.QmmError):
            g.string("v.u32")
        with pytest.raises(qmm.QmmError, match="no metadata key"):
            g.u64("missing")
        assert g.value_type("missing") == -1


def test_tensors_load_with_their_bytes(tmp_path):
    p = tmp_path / "t.gguf"
    tensors = sample_tensors()
    G.write(p, [("general.alignment", G.U32, 64)], tensors, alignment=64)
    H = qmm.host()
    with open_file(p) as g:
        assert g.tensor_data_offset % 64 == 0
        for name, dims, dtype, data in tensors:
            h = g.load_tensor(name, -1)
            try:
                assert H.qmm_qtensor_storage_bytes(h) == len(data)
            finally:
                H.qmm_qtensor_free(h)
    # the C++ writer's file, read by the Python reader: the same table and bytes
    out = tmp_path / "w.gguf"
    handles = []
    with open_file(p) as g:
        for name, *_ in tensors:
            handles.append((name, g.load_tensor(name, -1)))
    try:
        kv = G.kv_bytes(ALL_VALUES[:3], version=3)
        qmm.gguf_write(str(out), 3, kv, handles)
    finally:
        for _, h in handles:
            H.qmm_qtensor_free(h)
    version, meta, table, start = G.read(out)
    assert version == 2 and meta["general.architecture"] == (G.STRING, "llama") and meta["v.u8"] == (G.U8, 200)
    raw = open(out, "rb").read()
    for (name, dims, dtype, data), (n2, d2, t2, off) in zip(tensors, table):
        want_dims = [1] + dims if len(dims) == 1 else dims  # a 1-D tensor loads as one row
        assert (n2, d2, t2) == (name, want_dims, dtype)
        assert off % 32 == 0 and raw[start + off:start + off + len(data)] == data
    # and the C++ reader agrees with itself on the rewritten file
    with open_file(out) as g:
        assert [t[0] for t in g.tensors()] == [t[0] for t in tensors]


def test_summary_skips_long_arrays_and_keeps_the_rest(tmp_path):
    # gguf_file.rs tests::summary_skips_long_arrays_and_keeps_the_rest
    n = 65
    meta = [("tokenizer.tokens", G.ARRAY, (G.STRING, [f"token{i}" for i in range(n)])),
            ("tokenizer.scores", G.ARRAY, (G.F32, [float(i) for i in range(n)])),
            ("short", G.ARRAY, (G.U32, [1, 2])), ("general.name", G.STRING, "tiny")]
    p = tmp_path / "s.gguf"
    G.write(p, meta, [], version=2)
    with open_file(p, summary=True) as s, open_file(p) as full:
        assert s.value_type("tokenizer.tokens") == -1 and s.value_type("tokenizer.scores") == -1
        assert s.array("short")[0] == 2 and s.string("general.name") == "tiny"
        assert full.array("tokenizer.tokens")[0] == 65
        assert full.tensor_data_offset == s.tensor_data_offset


def test_long_fixed_size_arrays_are_located_not_parsed(tmp_path):
    # gguf_file.rs tests::long_fixed_size_arrays_are_located_not_parsed
    n = (1 << 20) + 3
    blob = [i % 251 for i in range(n)]
    meta = [("blob", G.ARRAY, (G.U8, blob)), ("short", G.ARRAY, (G.U64, [7, 9])), ("name", G.STRING, "probe")]
    p = tmp_path / "l.gguf"
    G.write(p, meta, [], version=2)
    with open_file(p) as g:
        assert g.value_type("blob") == -2
        assert g.array("short") == (2, G.U64) and g.string("name") == "probe"
        assert list(g.large_array("blob", n - 3, n, 1)) == blob[n - 3:]
        with pytest.raises(qmm.QmmError, match="outside"):
            g.large_array("blob", 0, n + 1, 1)


def test_peek_architecture(tmp_path):
    p = tmp_path / "a.gguf"
    G.write(p, ALL_VALUES, [])
    b = ctypes.create_string_buffer(64)
    assert qmm.host().qmm_gguf_peek_architecture(str(p).encode(), b, 64) == 0 and b.value == b"llama"
    G.write(p, ALL_VALUES[1:] + ALL_VALUES[:1], [])
    assert qmm.host().qmm_gguf_peek_architecture(str(p).encode(), b, 64) == 0 and b.value == b""


def _rejects(path, pattern):
    with pytest.raises(qmm.QmmError, match=pattern):
        qmm.GgufFile(str(path))


def test_malformed_files_are_rejected(tmp_path):
    p = tmp_path / "bad.gguf"
    G.write(p, ALL_VALUES, [], magic=0x12345678)
    _rejects(p, "unknown magic")
    G.write(p, ALL_VALUES, [], version=4)
    _rejects(p, "unsupported version")
    # truncated in the middle of the metadata
    G.write(p, ALL_VALUES, sample_tensors())
    raw = open(p, "rb").read()
    open(p, "wb").write(raw[:60])
    _rejects(p, "end of file|exceeds|needs at least")
    # counts that cannot fit in the file
    open(p, "wb").write(struct.pack("<IIQQ", 0x46554747, 3, 1000, 1000))
    _rejects(p, "needs at least")
    # a string longer than the rest of the file
    bad = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1 << 20) + b"k"
    open(p, "wb").write(bad + b"\0" * 32)
    _rejects(p, "string length")
    # a bool that is neither 0 nor 1
    G.write(p, [("b", G.BOOL, 0)], [], raw_kv=G._string("b", 3) + struct.pack("<IB", G.BOOL, 2))
    _rejects(p, "bool")
    # an unknown value type
    G.write(p, [("x", G.U8, 0)], [], raw_kv=G._string("x", 3) + struct.pack("<IB", 13, 0))
    _rejects(p, "value-type")
    # arrays nested deeper than 64
    v = (G.U8, [1])
    for _ in range(66):
        v = (G.ARRAY, [v])
    G.write(p, [("deep", G.ARRAY, v)], [])
    _rejects(p, "depth")
    # an array whose length exceeds what remains
    G.write(p, [("a", G.ARRAY, (G.U32, [1]))], [],
            raw_kv=G._string("a", 3) + struct.pack("<IIQ", G.ARRAY, G.U32, 10 ** 6) + b"\0" * 8)
    _rejects(p, "array of")
    # too many tensor dimensions
    G.write(p, [], [("t", [1] * 9, 0, b"\0" * 4)])
    _rejects(p, "dimensions")
    # an unknown tensor type fails Content::read
    G.write(p, [], [("t", [32], 99, b"\0" * 64)])
    _rejects(p, "unknown dtype")


def test_tensor_reads_are_bounded(tmp_path):
    p = tmp_path / "b.gguf"
    data = qbytes(O.Q4K, 2, 256, 5)
    G.write(p, [], [("w", [2, 256], O.Q4K, data)])
    raw = open(p, "rb").read()
    open(p, "wb").write(raw[:-10])  # the tensor's last bytes are missing
    with open_file(p) as g:
        with pytest.raises(qmm.QmmError, match="remaining in file"):
            g.load_tensor("w", -1)
        with pytest.raises(qmm.QmmError, match="cannot find"):
            g.load_tensor("nope", -1)
    G.write(p, [], [("w", [3, 100], O.Q8_0, b"\0" * 400)])  # 300 values: not whole Q8_0 blocks
    with open_file(p) as g:
        with pytest.raises(qmm.QmmError, match="divisible"):
            g.load_tensor("w", -1)
