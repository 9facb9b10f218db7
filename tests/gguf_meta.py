"""Test-side GGUF metadata reader (key -> value), written from the public GGUF
layout (little endian: magic, version, tensor count, kv count, then typed
key/value pairs), independent of the product's reader."""
from __future__ import annotations

import struct

_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def read_metadata(path: str) -> dict:
    with open(path, "rb") as f:
        data = f.read(64 << 20)   # metadata sits at the front of the file
    if data[:4] != b"GGUF":
        raise ValueError("not a GGUF file")
    pos = 8
    _n_tensors, n_kv = struct.unpack_from("<QQ", data, pos)
    pos += 16

    def string():
        nonlocal pos
        (n,) = struct.unpack_from("<Q", data, pos)
        pos += 8
        s = data[pos:pos + n]
        pos += n
        return s.decode("utf-8")

    def value(t):
        nonlocal pos
        if t == 8:
            return string()
        if t == 9:
            et, n = struct.unpack_from("<IQ", data, pos)
            pos += 12
            return [value(et) for _ in range(n)]
        fmt = _SCALARS[t]
        (v,) = struct.unpack_from(fmt, data, pos)
        pos += struct.calcsize(fmt)
        return v

    meta = {}
    for _ in range(n_kv):
        k = string()
        (t,) = struct.unpack_from("<I", data, pos)
        pos += 4
        meta[k] = value(t)
    return meta
