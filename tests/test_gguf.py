"""GGUF v3 reader of the library (sf37_hip_gguf_*, the engine's reader
sf37.c:506-604): offsets, sizes, types and dims of every tensor, the
alignment key, every key/value type skipped, and the malformed files the
reader must refuse.  Parsing needs no GPU."""
import ctypes as C
import struct

import numpy as np
import pytest

from gguf_writer import T_BF16, T_F32, T_Q2D, T_Q3GU, T_Q8_0, gguf_bytes


@pytest.fixture(scope="module")
def L():
    from sf37_amd import hip
    return hip.lib()


KVS = [("general.architecture", "str", "sf37"), ("general.alignment", "u32", 64), ("a.u8", "u8", 7),
       ("a.i8", "i8", -3), ("a.u16", "u16", 9), ("a.i16", "i16", -9), ("a.i32", "i32", -5), ("a.f32", "f32", 1.5),
       ("a.bool", "bool", 1), ("a.u64", "u64", 1 << 40), ("a.i64", "i64", -(1 << 40)), ("a.f64", "f64", 2.5),
       ("a.arr_u32", "arr", ("u32", [1, 2, 3])), ("a.arr_str", "arr", ("str", ["x", "yz"])),
       ("a.arr_arr", "arr", ("arr", [("u8", [1, 2]), ("u8", [3])]))]


def sample_tensors():
    r = np.random.default_rng(5)
    return [("t.f32", (8, 3), T_F32, r.standard_normal(24).astype(np.float32).tobytes()),
            ("t.bf16", (16,), T_BF16, r.integers(0, 1 << 16, 16).astype(np.uint16).tobytes()),
            ("t.q8", (64, 2), T_Q8_0, r.integers(0, 256, 4 * 34).astype(np.uint8).tobytes()),
            ("t.q3", (256, 2, 3), T_Q3GU, r.integers(0, 256, 6 * 110).astype(np.uint8).tobytes()),
            ("t.q2", (512, 1, 2), T_Q2D, r.integers(0, 256, 4 * 84).astype(np.uint8).tobytes()),
            ("t.other", (32,), 2, bytes(18))]   # a type the MoE path does not read: listed with 0 bytes


def lookup(L, g, name):
    off, nb, ty, nd = C.c_uint64(), C.c_uint64(), C.c_uint32(), C.c_uint32()
    dims = (C.c_uint64 * 4)()
    ok = L.sf37_hip_gguf_tensor(g, name.encode(), C.byref(off), C.byref(nb), C.byref(ty), C.byref(nd), dims)
    return ok, off.value, nb.value, ty.value, nd.value, tuple(dims)


def test_parse_offsets_types_dims(L, tmp_path):
    tensors = sample_tensors()
    data, start, offs = gguf_bytes(KVS, tensors, alignment=64)
    assert start % 64 == 0
    path = tmp_path / "m.gguf"
    path.write_bytes(data)
    g = L.sf37_hip_gguf_open(str(path).encode())
    assert g
    try:
        size = C.c_uint64()
        base = L.sf37_hip_gguf_map(g, C.byref(size))
        assert size.value == len(data)
        mapped = C.string_at(base, size.value)
        for (name, dims, typ, raw), rel in zip(tensors, offs):
            ok, off, nb, ty, nd, d4 = lookup(L, g, name)
            assert ok and off == start + rel and ty == typ and nd == len(dims)
            assert d4 == tuple(dims) + (1,) * (4 - len(dims))
            if typ == 2:
                assert nb == 0
            else:
                assert nb == len(raw) and mapped[off:off + nb] == raw
        assert lookup(L, g, "absent")[0] == 0
    finally:
        L.sf37_hip_gguf_close(g)


def test_from_map_default_alignment(L):
    tensors = sample_tensors()[:3]
    data, start, offs = gguf_bytes([("x", "str", "y")], tensors, alignment=32)
    buf = C.create_string_buffer(data, len(data))
    g = L.sf37_hip_gguf_from_map(C.cast(buf, C.c_void_p), len(data))
    assert g
    try:
        for (name, _, _, raw), rel in zip(tensors, offs):
            ok, off, nb, _, _, _ = lookup(L, g, name)
            assert ok and off == start + rel and nb == len(raw)
    finally:
        L.sf37_hip_gguf_close(g)


def refused(L, data):
    buf = C.create_string_buffer(data, len(data))
    return not L.sf37_hip_gguf_from_map(C.cast(buf, C.c_void_p), len(data))


def test_refuses_malformed(L):
    good, start, _ = gguf_bytes(KVS, sample_tensors(), alignment=64)
    assert not refused(L, good)
    assert refused(L, b"GGUX" + good[4:])                              # magic
    assert refused(L, gguf_bytes(KVS, sample_tensors(), version=2)[0])  # version
    assert refused(L, good[:40])                                        # truncated key/values
    assert refused(L, good[:start - 8])                                 # truncated tensor table
    big = [("t.f32", (8, 3), T_F32, bytes(96))]
    d, s, _ = gguf_bytes([], big)
    assert refused(L, d[:-4])                                           # data past the end
    # a tensor with rank 0
    r0 = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + struct.pack("<Q", 1) + b"t" + struct.pack("<IIQ", 0, 0, 0)
    assert refused(L, r0 + bytes(64))
    # an unknown key/value type
    kv = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 99) + bytes(16)
    assert refused(L, kv)
