"""Minimal pure-Python GGUF v3 reader (metadata, tensor infos, raw tensor bytes).

Independent of the C++ reader in csrc/gguf.cpp; used by tests and benchmarks."""
from __future__ import annotations

import mmap
import struct
from pathlib import Path

SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def read_gguf(path: str | Path):
    with open(path, "rb") as f:
        data = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
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


def tensor_bytes(path: str | Path, name: str) -> tuple[bytes, dict]:
    """Raw GGUF bytes of one tensor and its info (ne, type)."""
    import numpy as np

    _, _, tensors, data = read_gguf(path)
    t = tensors[name]
    n = 1
    for d in t["ne"]:
        n *= d
    from . import type_bytes

    nb = type_bytes(t["type"], n)
    return np.frombuffer(data, dtype=np.uint8, count=nb, offset=t["data_start"]), t
