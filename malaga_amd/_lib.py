"""ctypes binding of libmalaga_hip.so (declarations in include/malaga_hip.h).

The library is built in-tree by ``malaga_amd/build.py`` (hipcc for gfx950).
Loading fails loudly if it is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "_build" / "libmalaga_hip.so"

OK, ERR_INVALID, ERR_OOM, ERR_HIP, ERR_IO, ERR_FORMAT, ERR_UNSUPPORTED, ERR_NO_DEVICE = range(8)
F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 8, 12, 13, 14, 30
PRESETS = {"f32": 0, "f16": 1, "q8_0": 2, "q6_k": 3, "q5_k_m": 4, "q4_k_m": 5}
INIT_TESTUTIL, INIT_NORMAL, INIT_NORMAL_RICH = 0, 1, 2
FLAG_EOS_MASK, FLAG_NO_GRAPH = 1, 2


class MalagaError(RuntimeError):
    """Error raised for a non-zero status; ``code`` is the MLG_ERR_* value."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class Config(C.Structure):
    """src/config.rs:14-39, field for field."""

    _fields_ = [(n, C.c_int) for n in (
        "vocab_size", "d_model", "encoder_layers", "decoder_layers", "encoder_heads", "decoder_heads",
        "encoder_ffn", "decoder_ffn", "max_position_embeddings", "max_length", "scale_embedding",
        "bos_token_id", "pad_token_id", "eos_token_id", "decoder_start_token_id")]

    def as_dict(self) -> dict:
        return {n: getattr(self, n) for n, _ in self._fields_}


class CGenOptions(C.Structure):
    _fields_ = [("beam_size", C.c_int), ("max_new_tokens", C.c_int), ("length_penalty", C.c_float),
                ("sync_every", C.c_int), ("max_batch", C.c_int), ("fused", C.c_int), ("flags", C.c_uint32),
                ("shortlist", C.c_char_p)]


class ShortlistSpec(C.Structure):
    _fields_ = [("code", C.c_char_p), ("lang_id", C.c_uint32), ("ids", C.POINTER(C.c_uint32)), ("n_ids", C.c_int)]


TENSOR_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_char_p, C.c_int64, C.POINTER(C.c_float))
# mlg_beam_decode_fn(user, step, rows, reorder, next, vals, idx)
BEAM_DECODE_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                             C.POINTER(C.c_float), C.POINTER(C.c_uint32))

_P = C.c_void_p
_u32p = C.POINTER(C.c_uint32)
_intp = C.POINTER(C.c_int)
_fp = C.POINTER(C.c_float)

# name -> (restype, argtypes)
SIGNATURES = {
    "mlg_last_error": (C.c_char_p, []),
    "mlg_version": (C.c_char_p, []),
    "mlg_type_info": (C.c_int, [C.c_uint32, _intp, _intp]),
    "mlg_type_bytes": (C.c_int64, [C.c_uint32, C.c_int64]),
    "mlg_quantize": (C.c_int, [C.c_uint32, _P, C.c_int64, _P]),
    "mlg_dequantize": (C.c_int, [C.c_uint32, _P, C.c_int64, _P]),
    "mlg_preset_from_name": (C.c_int, [C.c_char_p, _intp]),
    "mlg_convert": (C.c_int, [C.c_char_p, C.POINTER(Config), C.c_int, C.c_char_p, C.c_char_p, TENSOR_FN, _P]),
    "mlg_write_synthetic": (C.c_int, [C.c_char_p, C.POINTER(Config), C.c_int, C.c_int, C.c_uint64, C.c_float,
                                      C.c_char_p]),
    "mlg_convert_sl": (C.c_int, [C.c_char_p, C.POINTER(Config), C.c_int, C.c_char_p, C.c_char_p, TENSOR_FN, _P,
                                 C.POINTER(ShortlistSpec), C.c_int]),
    "mlg_write_synthetic_sl": (C.c_int, [C.c_char_p, C.POINTER(Config), C.c_int, C.c_int, C.c_uint64, C.c_float,
                                         C.c_char_p, C.POINTER(ShortlistSpec), C.c_int]),
    "mlg_tiny_config": (None, [C.POINTER(Config)]),
    "mlg_device_count": (C.c_int, [_intp]),
    "mlg_ctx_create": (C.c_int, [C.c_int, C.POINTER(_P)]),
    "mlg_ctx_destroy": (None, [_P]),
    "mlg_model_load": (C.c_int, [_P, C.c_char_p, C.POINTER(_P)]),
    "mlg_model_free": (None, [_P]),
    "mlg_model_config": (C.c_int, [_P, C.POINTER(Config)]),
    "mlg_model_weight_bytes": (C.c_int64, [_P]),
    "mlg_model_shortlist_count": (C.c_int, [_P]),
    "mlg_model_shortlist_info": (C.c_int, [_P, C.c_int, C.POINTER(C.c_char_p), _intp]),
    "mlg_gen_options_default": (None, [C.POINTER(CGenOptions)]),
    "mlg_generate": (C.c_int, [_P, _P, _P, C.c_int, C.c_uint32, C.POINTER(CGenOptions), _P, C.c_int, _P]),
    "mlg_encode": (C.c_int, [_P, _P, _P, C.c_int, C.POINTER(_P)]),
    "mlg_batch_free": (None, [_P]),
    "mlg_greedy": (C.c_int, [_P, _P, C.c_uint32, C.c_int, C.c_int, C.c_uint32, _P, C.c_int, _P]),
    "mlg_greedy_top": (C.c_int, [_P, _P, C.c_uint32, C.c_int, C.c_int, C.c_uint32, _P, _P, C.c_int, _P]),
    "mlg_greedy_sl": (C.c_int, [_P, _P, C.c_uint32, C.c_char_p, C.c_int, C.c_int, C.c_uint32, _P, C.c_int, _P]),
    "mlg_beam": (C.c_int, [_P, _P, C.c_uint32, C.c_int, C.c_int, C.c_float, C.c_uint32, _P, C.c_int, _P]),
    "mlg_beam_search_host": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_float, C.c_uint32, BEAM_DECODE_FN, _P, _P,
                                       C.c_int, _P]),
    "mlg_server_start": (C.c_int, [_P, C.POINTER(CGenOptions), C.POINTER(_P)]),
    "mlg_server_stop": (None, [_P]),
    "mlg_server_submit": (C.c_int, [_P, _P, _P, C.c_int, C.c_uint32, C.c_uint32, C.c_int, C.c_char_p,
                                    C.POINTER(_P)]),
    "mlg_job_wait": (C.c_int, [_P, C.c_int, _intp]),
    "mlg_job_result": (C.c_int, [_P, _P, C.c_int, _P]),
    "mlg_job_free": (None, [_P]),
    "mlg_server_stats": (C.c_int, [_P, C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                                   C.POINTER(C.c_int64)]),
    "mlg_clear_graphs": (None, [_P]),
    "mlg_graph_stats": (C.c_int, [_P, _intp, _intp, _intp]),
    "mlg_graph_cache_keys": (C.c_int, [_P, _P, C.c_int]),
    "mlg_debug_fail_alloc_after": (None, [C.c_long]),
    "mlg_debug_tile_major": (C.c_int64, [C.c_uint32, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int64]),
    "mlg_bench_stream_read": (C.c_int, [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "mlg_matrix_upload": (C.c_int, [_P, C.c_uint32, C.c_int, C.c_int, _P, C.POINTER(_P)]),
    "mlg_matrix_free": (None, [_P]),
    "mlg_matrix_bytes": (C.c_int64, [_P]),
    "mlg_gemv": (C.c_int, [_P, _P, C.c_int, _P, _P, C.c_int, _P]),
    "mlg_gemv_max_batch": (C.c_int, [_P]),
    "mlg_gemm": (C.c_int, [_P, _P, C.c_int, _P, _P, C.c_int, _P]),
    "mlg_gemm_resid": (C.c_int, [_P, _P, C.c_int, _P, _P, C.c_int, _P, _P]),
    "mlg_gemm_argmax_parts": (C.c_int, [_P, C.c_int]),
    "mlg_gemm_argmax": (C.c_int, [_P, _P, C.c_int, C.c_int, _P, _P, _P]),
    "mlg_gemv_argmax_parts": (C.c_int, [_P, C.c_int]),
    "mlg_gemv_argmax": (C.c_int, [_P, _P, C.c_int, C.c_int, _P, _P, _P]),
    "mlg_residual_ln": (C.c_int, [_P, _P, C.c_int, C.c_int, _P, _P, C.c_float, _P, _P]),
    "mlg_layernorm": (C.c_int, [_P, C.c_int, C.c_int, _P, _P, C.c_float, _P, _P]),
    "mlg_attn_decode": (C.c_int, [_P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P]),
    "mlg_argmax_partial": (C.c_int, [_P, C.c_int, C.c_int, C.c_int, _P, _P, C.c_int, _P]),
    "mlg_greedy_finalize": (C.c_int, [_P, _P, C.c_int, C.c_int, _P, _P, _P, C.c_int, _P, C.c_uint32, C.c_uint32,
                                      _P]),
    "mlg_logsoftmax_topk_scratch": (C.c_size_t, [C.c_int, C.c_int]),
    "mlg_logsoftmax_topk": (C.c_int, [_P, C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P]),
    "mlg_logsoftmax_topk_noalloc": (C.c_int, [_P, C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P]),
    "mlg_teacher_forced_logits": (C.c_int, [_P, _P, _P, C.c_int, _P, C.c_int, C.c_int, _P]),
    "mlg_bucket": (C.c_int, [C.c_int, C.c_int, C.c_int]),
    "mlg_budget": (C.c_int, [_P, C.c_int, C.c_int]),
    "mlg_synchronize": (C.c_int, []),
}

_lib = None


def lib_path() -> Path:
    return Path(os.environ.get("MALAGA_HIP_LIB", LIB_PATH))


def load(build_if_missing: bool = True) -> C.CDLL:
    """Loads libmalaga_hip.so (building it first if it is absent)."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not path.exists() and build_if_missing:
        from . import build as _build
        _build.build_library()
    if not path.exists():
        raise MalagaError(ERR_NO_DEVICE, f"{path} is missing: build it with malaga_amd.build.build_library()")
    lib = C.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != OK:
        msg = load().mlg_last_error()
        raise MalagaError(status, msg.decode() if msg else "")
