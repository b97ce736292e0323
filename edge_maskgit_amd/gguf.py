"""GGUF v3 file writer (the format the reference's converter writes and its loader reads:
tools/convert_to_gguf.py:127-266, src/mg-model.cpp:139-201).

write_gguf(path, meta, tensors) lays out the header, `key / type / value` metadata, tensor
infos with dims innermost-first (the reversed numpy shape), and 32-byte aligned data. It writes
given bytes only; quantizing weights into Q8_0 / Q4_K blocks is the caller's business.
"""
from __future__ import annotations

import struct

GGML_F32, GGML_Q8_0, GGML_Q4_K = 0, 8, 12
_U32, _I32, _F32, _STR, _ARRAY = 4, 5, 6, 8, 9
ALIGN = 32

def _s(b: bytearray, text: str):
    raw = text.encode()
    b += struct.pack("<Q", len(raw)) + raw


def write_gguf(path: str, meta: list, tensors: list) -> None:
    """meta: [(key, kind, value)] with kind in {"u32", "i32", "f32", "str", "i32_array"};
    tensors: [(name, numpy shape, ggml type, raw bytes)]."""
    kv = bytearray()
    for key, kind, val in meta:
        _s(kv, key)
        if kind == "u32":
            kv += struct.pack("<II", _U32, val)
        elif kind == "i32":
            kv += struct.pack("<Ii", _I32, val)
        elif kind == "f32":
            kv += struct.pack("<If", _F32, val)
        elif kind == "i32_array":       # array type, element type, count, elements
            kv += struct.pack("<IIQ", _ARRAY, _I32, len(val)) + struct.pack(f"<{len(val)}i", *val)
        else:
            kv += struct.pack("<I", _STR)
            _s(kv, val)
    info = bytearray()
    offsets, off = [], 0
    for name, shape, gtype, data in tensors:
        offsets.append(off)
        off = (off + len(data) + ALIGN - 1) // ALIGN * ALIGN
    for (name, shape, gtype, data), o in zip(tensors, offsets):
        _s(info, name)
        info += struct.pack("<I", len(shape))
        for d in reversed(shape):
            info += struct.pack("<Q", int(d))
        info += struct.pack("<IQ", gtype, o)
    head = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(meta)) + kv + info
    pad = (-len(head)) % ALIGN
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        pos = 0
        for (name, shape, gtype, data), o in zip(tensors, offsets):
            f.write(b"\0" * (o - pos))
            f.write(data)
            pos = o + len(data)
