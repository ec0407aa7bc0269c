"""The C ABI: libmalaga_hip.so loads, exports every declared symbol, and fails loudly without a GPU."""
import ctypes
import re
from pathlib import Path

import pytest

import malaga_amd as M
from malaga_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "malaga_hip.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mlg_\w+)\s*\(", text)) - {"mlg_tensor_fn"})


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(str(_lib.lib_path()))
    names = declared()
    assert len(names) > 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing


def test_python_binding_covers_the_header():
    assert set(declared()) <= set(_lib.SIGNATURES)


def test_no_device_is_a_loud_error():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(M.MalagaError) as e:
        M.Translator.load("/nonexistent.gguf")
    assert e.value.code == _lib.ERR_NO_DEVICE


def test_unknown_preset_is_an_error():
    n = ctypes.c_int()
    assert _lib.load().mlg_preset_from_name(b"q4_0", ctypes.byref(n)) == _lib.ERR_INVALID
    assert b"q4_k_m" in _lib.load().mlg_last_error()


def test_q6k_tile_major_copy_holds_what_each_lane_reads():
    """The decode GEMMs' tile-major q6_K copy, checked against the GGUF q6_K block format
    (ql[128] | qh[64] | int8 scales[16] | f16 d per 256 values): lane 16 kq + r of tile t
    finds, for K block kb, ql[64 n + 16 h + 4 kq .. +4] (piece 0), ql[64 n + 32 + 16 h + 4 kq
    .. +4] (piece 1) and qh[32 n + 16 h + 4 kq .. +4] (piece 2) as dword 2 n + h of its
    16-byte piece, then row 16 t + r's scales and d.  Every quant byte is read exactly once;
    the rows that pad N to a multiple of 16 are zero."""
    import numpy as np

    lib = _lib.load()
    N, K = 40, 768
    nb = K // 256
    rng = np.random.default_rng(7)
    rows = rng.integers(0, 256, size=(N, nb, 210), dtype=np.uint8)
    src = np.ascontiguousarray(rows)
    size = lib.mlg_debug_tile_major(14, N, K, src.ctypes.data, None, 0)
    assert size == 3 * nb * 3456
    out = np.zeros(size, dtype=np.uint8)
    assert lib.mlg_debug_tile_major(14, N, K, src.ctypes.data, out.ctypes.data, size) == size
    # no tile-major form: other types, K not a whole number of q6_K blocks
    assert lib.mlg_debug_tile_major(8, N, K, src.ctypes.data, None, 0) == 0  # q8_0
    assert lib.mlg_debug_tile_major(14, N, 128, src.ctypes.data, None, 0) == 0
    seen = np.zeros((N, nb, 192), dtype=np.int32)
    for t in range(3):
        for kb in range(nb):
            tb = out[(t * nb + kb) * 3456:(t * nb + kb + 1) * 3456]
            for r in range(16):
                if 16 * t + r >= N:
                    for piece in range(3):
                        for kq in range(4):
                            lane = 16 * kq + r
                            assert not tb[1024 * piece + 16 * lane:1024 * piece + 16 * lane + 16].any()
                    assert not tb[3072 + 16 * r:3088 + 16 * r].any() and not tb[3328 + 2 * r:3330 + 2 * r].any()
                    continue
                blk = rows[16 * t + r, kb]
                for kq in range(4):
                    lane = 16 * kq + r
                    for n in range(2):
                        for h in range(2):
                            dw = 4 * (2 * n + h)
                            for piece, off in ((0, 64 * n + 16 * h + 4 * kq), (1, 64 * n + 32 + 16 * h + 4 * kq),
                                               (2, 128 + 32 * n + 16 * h + 4 * kq)):
                                got = tb[1024 * piece + 16 * lane + dw:1024 * piece + 16 * lane + dw + 4]
                                assert (got == blk[off:off + 4]).all()
                                seen[16 * t + r, kb, off:off + 4] += 1
                assert (tb[3072 + 16 * r:3088 + 16 * r] == blk[192:208]).all()
                assert (tb[3328 + 2 * r:3330 + 2 * r] == blk[208:210]).all()
            assert not tb[3360:].any()
    assert (seen == 1).all()


def test_q4k_tile_major_copy_holds_what_each_lane_reads():
    """The q4_K tile-major copy against the GGUF q4_K block (f16 d | f16 dmin | 12 bytes of
    packed scales | qs[128] per 256 values): row 16 t + r's 16-byte header at 16 r, and lane
    16 kq + r's 8-byte groups qs[32 g + 8 kq .. + 8] at 256 + 1024 (g / 2) + 16 lane + 8 (g % 2).
    Every qs byte is read exactly once; padding rows are zero."""
    import numpy as np

    lib = _lib.load()
    N, K = 24, 512
    nb = K // 256
    rows = np.random.default_rng(8).integers(0, 256, size=(N, nb, 144), dtype=np.uint8)
    size = lib.mlg_debug_tile_major(12, N, K, rows.ctypes.data, None, 0)
    assert size == 2 * nb * 2304
    out = np.zeros(size, dtype=np.uint8)
    assert lib.mlg_debug_tile_major(12, N, K, rows.ctypes.data, out.ctypes.data, size) == size
    seen = np.zeros((N, nb, 128), dtype=np.int32)
    for t in range(2):
        for kb in range(nb):
            tb = out[(t * nb + kb) * 2304:(t * nb + kb + 1) * 2304]
            for r in range(16):
                n = 16 * t + r
                for kq in range(4):
                    lane = 16 * kq + r
                    for g in range(4):
                        o = 256 + 1024 * (g // 2) + 16 * lane + 8 * (g % 2)
                        if n >= N:
                            assert not tb[o:o + 8].any()
                            continue
                        assert (tb[o:o + 8] == rows[n, kb, 16 + 32 * g + 8 * kq:24 + 32 * g + 8 * kq]).all()
                        seen[n, kb, 32 * g + 8 * kq:32 * g + 8 * kq + 8] += 1
                want = rows[n, kb, :16] if n < N else np.zeros(16, np.uint8)
                assert (tb[16 * r:16 * r + 16] == want).all()
    assert (seen == 1).all()
