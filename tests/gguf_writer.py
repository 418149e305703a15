"""Minimal GGUF v3 writer for test fixtures (the layout of the GGUF spec that
gguf-py's GGUFWriter produces for convert/convert_thinksound.py and
convert/quantize_gguf.py): header, metadata, tensor infos, tensor data
aligned to `general.alignment` (32). Written from the published format, for
the loader tests; the converters themselves are not used."""
import struct

import numpy as np

U32, I32, F32, BOOL, STRING = 4, 5, 6, 7, 8
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, kv, tensors, alignment=32):
    """kv: {key: (type, value)}; tensors: [(name, ggml_ne tuple, ggml_type, raw bytes)]"""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv) + 1))
    items = dict(kv)
    items["general.alignment"] = (U32, alignment)
    for k, (t, v) in items.items():
        out += _str(k) + struct.pack("<I", t)
        if t == U32:
            out += struct.pack("<I", v)
        elif t == I32:
            out += struct.pack("<i", v)
        elif t == F32:
            out += struct.pack("<f", v)
        elif t == BOOL:
            out += struct.pack("<B", int(v))
        elif t == STRING:
            out += _str(v)
        else:
            raise ValueError(t)
    offsets, off = [], 0
    for name, ne, gt, raw in tensors:
        offsets.append(off)
        off += (len(raw) + alignment - 1) // alignment * alignment
    for (name, ne, gt, raw), o in zip(tensors, offsets):
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", gt, o)
    out += b"\0" * ((-len(out)) % alignment)
    for (name, ne, gt, raw), o in zip(tensors, offsets):
        out += raw + b"\0" * ((-len(raw)) % alignment)
    with open(path, "wb") as f:
        f.write(bytes(out))


def f32_tensor(name, arr):
    """numpy array (C order) -> ggml ne (reversed shape), F32 bytes"""
    arr = np.ascontiguousarray(arr, dtype=np.float32)
    return name, tuple(reversed(arr.shape)), GGML_F32, arr.tobytes()


def f16_tensor(name, arr):
    arr = np.ascontiguousarray(arr, dtype=np.float16)
    return name, tuple(reversed(arr.shape)), GGML_F16, arr.tobytes()


def bf16_tensor(name, bits):
    """bits: uint16 bf16 patterns"""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    return name, tuple(reversed(bits.shape)), GGML_BF16, bits.tobytes()


def q8_0_tensor(name, blocks, K):
    """blocks: uint8 [rows, K/32, 34] ggml Q8_0 blocks of rows of K values"""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    rows = blocks.shape[0]
    return name, (K, rows), GGML_Q8_0, blocks.tobytes()
