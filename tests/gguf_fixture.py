"""Synthetic GGUF v3 files for the pack-loader tests: a header, typed metadata (strings, integers and arrays, so the
readers skip every kind), a tensor directory and each tensor's payload filled with a recognisable byte pattern.
Written from the GGUF v3 layout: magic, version, tensor and key counts, key/values, then per tensor its name, n_dims,
dims (dim 0 the row), type and offset in the data section, which starts at the next multiple of general.alignment."""
import struct

import numpy as np

BLOCK = {7: (32, 24), 8: (32, 34), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 21: (256, 110),
         23: (256, 136), 42: (64, 18)}


def pattern(seed, start, n):
    """Payload bytes [start, start + n) of a tensor seeded `seed`."""
    i = np.arange(start, start + n, dtype=np.uint64)
    return ((np.uint64(seed) * np.uint64(37) + i * np.uint64(11) + (i >> np.uint64(10))) & np.uint64(0xFF)).astype(np.uint8)


def payload(t, shape):
    qk, b = BLOCK[t]
    n = 1
    for d in shape:
        n *= d
    return n // qk * b


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def write(path, tensors, kv=(), align=32, cut=0):
    """tensors: [(name, shape, type, seed)]; kv: [(key, type, value)] with type 8 string, 4 u32, 2 u16, 5 i32, 10 u64
    or (9, (elem_type, [values])).  Returns dict(data_start, offsets (from the data start), size)."""
    h = bytearray(struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kv) + (align != 32)))
    items = list(kv) + ([("general.alignment", 4, align)] if align != 32 else [])
    fmt = {4: "<I", 2: "<H", 5: "<i", 10: "<Q"}
    for key, t, v in items:
        h += _s(key) + struct.pack("<I", t)
        if t == 8:
            h += _s(v)
        elif t == 9:
            et, vals = v
            h += struct.pack("<IQ", et, len(vals))
            for x in vals:
                h += _s(x) if et == 8 else struct.pack(fmt[et], x)
        else:
            h += struct.pack(fmt[t], v)
    offs, at = [], 0
    for name, shape, t, seed in tensors:
        h += _s(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        h += struct.pack("<IQ", t, at)
        offs.append(at)
        at = (at + payload(t, shape) + align - 1) // align * align
    data_start = (len(h) + align - 1) // align * align
    h += b"\0" * (data_start - len(h))
    body = bytearray(at)
    for (name, shape, t, seed), o in zip(tensors, offs):
        n = payload(t, shape)
        body[o:o + n] = pattern(seed, 0, n).tobytes()
    data = bytes(h + body)
    if cut:
        data = data[:-cut]
    with open(path, "wb") as f:
        f.write(data)
    return dict(data_start=data_start, offsets=offs, size=len(data))
