"""Minimal GGUF v3 reader used by the tests (independent of the C++ reader)."""
from __future__ import annotations

import struct
from pathlib import Path

SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def read_gguf(path: str | Path):
    data = Path(path).read_bytes()
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, data, pos)
        pos += struct.calcsize(fmt)
        return v[0]

    def string():
        nonlocal pos
        n = take("<Q")
        s = data[pos: pos + n].decode()
        pos += n
        return s

    def value(t):
        if t == 8:
            return string()
        if t == 9:
            et, n = take("<I"), take("<Q")
            return [value(et) for _ in range(n)]
        return take(SCALAR[t])

    assert take("<I") == 0x46554747, "bad magic"
    version = take("<I")
    nt, nkv = take("<Q"), take("<Q")
    meta = {}
    for _ in range(nkv):
        k = string()
        meta[k] = value(take("<I"))
    tensors = {}
    for _ in range(nt):
        name = string()
        nd = take("<I")
        ne = [take("<Q") for _ in range(nd)]
        tensors[name] = dict(ne=ne, type=take("<I"), offset=take("<Q"))
    align = meta.get("general.alignment", 32)
    start = (pos + align - 1) // align * align
    for t in tensors.values():
        t["data_start"] = start + t["offset"]
    return version, meta, tensors, data
