"""Minimal GGUF v3 writer for tests (the container the engine reads,
sf37.c:506-604): key/value section, tensor table, aligned data section."""
import struct

import numpy as np

GV = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7, "str": 8, "arr": 9,
      "u64": 10, "i64": 11, "f64": 12}
FMT = {"u8": "<B", "i8": "<b", "u16": "<H", "i16": "<h", "u32": "<I", "i32": "<i", "f32": "<f", "bool": "<B",
       "u64": "<Q", "i64": "<q", "f64": "<d"}
T_F32, T_F16, T_Q8_0, T_Q2D, T_Q3GU, T_BF16 = 0, 1, 8, 10, 11, 30


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind, v):
    if kind == "str":
        return _str(v)
    if kind == "arr":
        ek, items = v
        return struct.pack("<IQ", GV[ek], len(items)) + b"".join(_value(ek, x) for x in items)
    return struct.pack(FMT[kind], v)


def gguf_bytes(kvs, tensors, alignment=32, version=3):
    """kvs: [(key, kind, value)]; tensors: [(name, dims (GGUF order), type, bytes)]."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for key, kind, v in kvs:
        head += _str(key) + struct.pack("<I", GV[kind]) + _value(kind, v)
    offs, pos = [], 0
    for _, _, _, data in tensors:
        pos = (pos + alignment - 1) // alignment * alignment
        offs.append(pos)
        pos += len(data)
    for (name, dims, typ, _), off in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", typ, off)
    start = (len(head) + alignment - 1) // alignment * alignment
    out = bytearray(head + b"\0" * (start - len(head)))
    for (_, _, _, data), off in zip(tensors, offs):
        out += b"\0" * (start + off - len(out))
        out += bytes(data)
    return bytes(out), start, offs


def moe_layer_tensors(il, router, router_type, router_bias, gate, up, down, sh_gate, sh_up, sh_down, norm_bits,
                      E, D, F, shared_q3q2=False):
    """The MoE tensors of layer il by the engine's contract (sf37.c:1760-1782);
    router is F32 / BF16 values or Q8_0 bytes; shared_q3q2: the shared expert
    in Q3GU (gate/up) and Q2D (down) instead of Q8_0."""
    p = f"model.layers.{il}."
    if router_type in (T_BF16, T_F16):
        rb = np.asarray(router, np.uint16).tobytes()
    elif router_type == T_Q8_0:
        rb = bytes(router)
    else:
        rb = np.asarray(router, np.float32).tobytes()
    sg, sd = (T_Q3GU, T_Q2D) if shared_q3q2 else (T_Q8_0, T_Q8_0)
    return [
        (p + "moe.gate.weight", (D, E), router_type, rb),
        (p + "moe.router_bias", (E,), T_F32, np.asarray(router_bias, np.float32).tobytes()),
        (p + "moe.gate_proj.weight", (D, F, E), T_Q3GU, gate),
        (p + "moe.up_proj.weight", (D, F, E), T_Q3GU, up),
        (p + "moe.down_proj.weight", (F, D, E), T_Q2D, down),
        (p + "share_expert.gate_proj.weight", (D, F), sg, sh_gate),
        (p + "share_expert.up_proj.weight", (D, F), sg, sh_up),
        (p + "share_expert.down_proj.weight", (F, D), sd, sh_down),
        (p + "post_attention_layernorm.weight", (D,), T_BF16, np.asarray(norm_bits, np.uint16).tobytes()),
    ]
