"""ctypes wrapper of the CPU oracle (oracle/oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the CPU
baseline timed by bench.py.  The product package (malaga_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path
from typing import Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"
REF_DIR = HERE / "_ref"

KV_F16, EOS_MASK = 1, 2


class OrcConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "vocab_size", "d_model", "encoder_layers", "decoder_layers", "encoder_heads", "decoder_heads",
        "encoder_ffn", "decoder_ffn", "max_position_embeddings", "max_length", "scale_embedding",
        "bos_token_id", "pad_token_id", "eos_token_id", "decoder_start_token_id")]


# orc_script_fn(user, step, rows, hist, hist_len, logprobs)
SCRIPT_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_uint32), C.c_int, C.POINTER(C.c_float))


class OrcGenOptions(C.Structure):
    _fields_ = [("beam_size", C.c_int), ("max_new_tokens", C.c_int), ("length_penalty", C.c_float),
                ("sync_every", C.c_int)]


_lib = None


def build(force: bool = False) -> Path:
    res = subprocess.run(["make", "-C", str(HERE)] + (["-B"] if force else []), capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building the oracle failed:\n{res.stdout}\n{res.stderr}")
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        P = C.c_void_p
        L.orc_last_error.restype = C.c_char_p
        L.orc_threads.restype, L.orc_threads.argtypes = C.c_int, []
        L.orc_h2f.restype, L.orc_h2f.argtypes = C.c_float, [C.c_uint16]
        L.orc_f2h.restype, L.orc_f2h.argtypes = C.c_uint16, [C.c_float]
        L.orc_dequant.restype, L.orc_dequant.argtypes = C.c_int, [C.c_uint32, P, C.c_int64, P]
        L.orc_gemv.restype, L.orc_gemv.argtypes = C.c_int, [C.c_uint32, P, C.c_int, C.c_int, P, C.c_int, P]
        L.orc_sinusoidal_table.restype, L.orc_sinusoidal_table.argtypes = None, [C.c_int, C.c_int, C.c_int, P]
        L.orc_load.restype, L.orc_load.argtypes = P, [C.c_char_p]
        L.orc_free.restype, L.orc_free.argtypes = None, [P]
        L.orc_get_config.restype, L.orc_get_config.argtypes = None, [P, C.POINTER(OrcConfig)]
        L.orc_encode.restype, L.orc_encode.argtypes = P, [P, P, P, C.c_int, C.c_int, C.c_int, P]
        L.orc_state_free.restype, L.orc_state_free.argtypes = None, [P]
        L.orc_decode.restype, L.orc_decode.argtypes = C.c_int, [P, P, P, C.c_int, P, P]
        L.orc_generate.restype = C.c_int
        L.orc_generate.argtypes = [P, P, P, C.c_int, C.c_uint32, C.POINTER(OrcGenOptions), C.c_int, P, C.c_int, P, P]
        L.orc_beam_scripted.restype = C.c_int
        L.orc_beam_scripted.argtypes = [C.c_int, C.c_int, C.c_int, C.c_uint32, C.c_int, C.c_float, C.c_int, SCRIPT_FN,
                                        P, C.c_int, P, P]
        L.orc_generate_sl.restype = C.c_int
        L.orc_generate_sl.argtypes = [P, P, P, C.c_int, C.c_uint32, C.POINTER(OrcGenOptions), C.c_int, P, C.c_int,
                                      P, C.c_int, P, P]
        _lib = L
    return _lib


def _err(msg: str):
    e = lib().orc_last_error()
    raise RuntimeError(f"{msg}: {e.decode() if e else ''}")


def threads() -> int:
    """OpenMP threads of the oracle's parallel regions."""
    return int(lib().orc_threads())


def h2f(bits: int) -> float:
    return float(lib().orc_h2f(bits))


def f2h(x: float) -> int:
    return int(lib().orc_f2h(x))


def dequant(ggml_type: int, blocks: np.ndarray, n: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n, dtype=np.float32)
    if lib().orc_dequant(ggml_type, b.ctypes.data, n, out.ctypes.data):
        _err("dequant")
    return out


def gemv(ggml_type: int, w_rows: np.ndarray, N: int, K: int, x: np.ndarray) -> np.ndarray:
    """y[r][n] = sum_k x[r][k] w[n][k] on raw GGUF rows (f64 accumulation)."""
    w = np.ascontiguousarray(w_rows, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    y = np.zeros((x.shape[0], N), dtype=np.float32)
    if lib().orc_gemv(ggml_type, w.ctypes.data, N, K, x.ctypes.data, x.shape[0], y.ctypes.data):
        _err("gemv")
    return y


def sinusoidal_table(n: int, dim: int, padding_idx: int) -> np.ndarray:
    out = np.zeros((n, dim), dtype=np.float32)
    lib().orc_sinusoidal_table(n, dim, padding_idx, out.ctypes.data)
    return out


def _flat(src: Sequence[Sequence[int]]):
    lens = np.array([len(r) for r in src], dtype=np.uint32)
    ids = np.array([t for r in src for t in r], dtype=np.uint32)
    return np.ascontiguousarray(ids), np.ascontiguousarray(lens)


class Model:
    """The dequantized f32 model of a GGUF file (src/model.rs semantics)."""

    def __init__(self, path: str | Path):
        self.L = lib()
        self.h = self.L.orc_load(str(path).encode())
        if not self.h:
            _err(f"loading {path}")
        c = OrcConfig()
        self.L.orc_get_config(self.h, C.byref(c))
        self.cfg = {n: getattr(c, n) for n, _ in c._fields_}

    def __del__(self):
        if getattr(self, "h", None):
            self.L.orc_free(self.h)
            self.h = None

    def budget(self, n: int, max_new_tokens: int | None = None) -> int:
        c = self.cfg
        cap = min(c["max_length"], c["max_position_embeddings"] - 2)
        v = max_new_tokens if max_new_tokens else 2 * n + 16
        return max(1, min(v, cap))

    def generate(self, src: Sequence[Sequence[int]], tgt_lang: int, beam_size: int = 1,
                 max_new_tokens: int | None = None, length_penalty: float = 1.0, sync_every: int = 4,
                 kv_f16: bool = True, eos_mask: bool = False,
                 shortlist: Sequence[int] | None = None) -> tuple[list[list[int]], float]:
        """One batch of src/translator.rs:175-207.  Returns (rows, min top-1/top-2 logit gap).
        ``shortlist``: sorted vocabulary ids of the target language's reduced LM head (greedy
        only); source tokens stay candidates (the fused shortlist step, src/model.rs:594-603)."""
        ids, lens = _flat(src)
        o = OrcGenOptions(beam_size, max_new_tokens or 0, length_penalty, sync_every)
        cap = max(self.budget(len(r), max_new_tokens) for r in src)
        out = np.zeros((len(src), cap), dtype=np.uint32)
        out_len = np.zeros(len(src), dtype=np.int32)
        gap = C.c_float(float("inf"))
        flags = (KV_F16 if kv_f16 else 0) | (EOS_MASK if eos_mask else 0)
        if shortlist is not None:
            sl = np.ascontiguousarray(np.asarray(shortlist, dtype=np.uint32))
            rc = self.L.orc_generate_sl(self.h, ids.ctypes.data, lens.ctypes.data, len(src), tgt_lang, C.byref(o),
                                        flags, sl.ctypes.data, int(sl.size), out.ctypes.data, cap,
                                        out_len.ctypes.data, C.byref(gap))
        else:
            rc = self.L.orc_generate(self.h, ids.ctypes.data, lens.ctypes.data, len(src), tgt_lang, C.byref(o),
                                     flags, out.ctypes.data, cap, out_len.ctypes.data, C.byref(gap))
        if rc:
            _err("generate")
        return [out[i, : out_len[i]].tolist() for i in range(len(src))], gap.value

    def translate_batch(self, src: Sequence[Sequence[int]], tgt_lang: int, max_batch: int = 32, **kw):
        """src/translator.rs:136-167: length-sorted batches (stable), results in input order."""
        order = sorted(range(len(src)), key=lambda i: -len(src[i]))
        out: list = [None] * len(src)
        gaps = []
        for k in range(0, len(order), max_batch):
            chunk = order[k: k + max_batch]
            rows, gap = self.generate([src[i] for i in chunk], tgt_lang, **kw)
            gaps.append(gap)
            for i, r in zip(chunk, rows):
                out[i] = r
        return out, min(gaps) if gaps else float("inf")

    def encoder_output(self, src: Sequence[Sequence[int]]) -> np.ndarray:
        ids, lens = _flat(src)
        s = int(lens.max())
        out = np.zeros((len(src), s, self.cfg["d_model"]), dtype=np.float32)
        st = self.L.orc_encode(self.h, ids.ctypes.data, lens.ctypes.data, len(src), 4, 0, out.ctypes.data)
        if not st:
            _err("encode")
        self.L.orc_state_free(st)
        return out

    def teacher_forced_logits(self, src: Sequence[Sequence[int]], tgt: np.ndarray, kv_f16: bool = True,
                              step_by_step: bool = True) -> np.ndarray:
        """Logits [n, T, vocab] after feeding tgt[:, t] at position t (one position per call
        when step_by_step, else all T positions in one causal pass, src/model.rs:515-536)."""
        ids, lens = _flat(src)
        tgt = np.ascontiguousarray(tgt, dtype=np.uint32)
        n, T = tgt.shape
        V = self.cfg["vocab_size"]
        st = self.L.orc_encode(self.h, ids.ctypes.data, lens.ctypes.data, n, T, KV_F16 if kv_f16 else 0, None)
        if not st:
            _err("encode")
        out = np.zeros((n, T, V), dtype=np.float32)
        try:
            if step_by_step:
                buf = np.zeros((n, V), dtype=np.float32)
                for t in range(T):
                    col = np.ascontiguousarray(tgt[:, t])
                    if self.L.orc_decode(self.h, st, col.ctypes.data, 1, buf.ctypes.data, None):
                        _err("decode")
                    out[:, t] = buf
            else:
                raise ValueError("only the last position's logits are returned by a multi-token pass")
        finally:
            self.L.orc_state_free(st)
        return out
