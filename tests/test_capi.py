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
