"""MI355X (gfx950) backend for malaga's NLLB/M2M100 GGUF decode path.

Host-side mirror of the reference interface (rzafiamy/malaga, crates/malaga-core):

  * ``GenOptions``           <- src/translator.rs:15-53
  * ``Translator.load``      <- src/translator.rs:62-73 (GGUF -> weights in HBM)
  * ``Translator.generate``  <- src/translator.rs:169-207 (token ids in, token ids out)
  * ``Translator.translate_batch_ids`` <- src/translator.rs:136-167 (sort, batch, OOM halving)
  * ``Translator.encode_cross`` / ``greedy`` / ``beam`` <- src/model.rs:463-477,
    src/graph.rs:204-223, src/translator.rs:250-335
  * ``convert`` / ``write_synthetic`` <- src/convert.rs:196-318, src/testutil.rs:16-101

Text tokenization and segmentation are outside this backend: callers pass
token ids, as ``Translator::generate`` does.  Every call goes to the HIP
library; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import json
from pathlib import Path
from typing import Callable, Sequence

import numpy as np

from ._lib import (FLAG_EOS_MASK, FLAG_NO_GRAPH, INIT_NORMAL, INIT_NORMAL_RICH, INIT_TESTUTIL, PRESETS, TENSOR_FN,
                   CGenOptions, Config, MalagaError, check, load)

__all__ = ["GenOptions", "Translator", "Server", "Job", "Config", "MalagaError", "convert", "write_synthetic", "tiny_config",
           "nllb_600m_config", "nllb_3b_config", "quantize", "dequantize", "type_bytes", "bucket",
           "INIT_TESTUTIL", "INIT_NORMAL", "INIT_NORMAL_RICH", "PRESETS"]


@dataclasses.dataclass
class GenOptions:
    """src/translator.rs:15-53.  ``shortlist`` (``--fast-vocab``): True uses the target
    language's shortlist (its code comes from the tokenizer, as the reference derives
    it); a string names the shortlist's language code directly; None decodes exactly."""

    beam_size: int = 1
    max_new_tokens: int | None = None
    length_penalty: float = 1.0
    sync_every: int = 4
    max_batch: int = 32
    fused: bool = True
    eos_mask: bool = False  # benchmark-only: EOS never chosen, so lengths are fixed
    shortlist: str | bool | None = None

    def _c(self) -> CGenOptions:
        o = CGenOptions()
        o.beam_size = self.beam_size
        o.max_new_tokens = self.max_new_tokens or 0
        o.length_penalty = self.length_penalty
        o.sync_every = self.sync_every
        o.max_batch = self.max_batch
        o.fused = 1 if self.fused else 0
        o.flags = FLAG_EOS_MASK if self.eos_mask else 0
        o.shortlist = self.shortlist.encode() if isinstance(self.shortlist, str) and self.shortlist else None
        return o


def _flat(src: Sequence[Sequence[int]]):
    lens = np.array([len(r) for r in src], dtype=np.uint32)
    ids = np.array([t for r in src for t in r], dtype=np.uint32) if len(src) else np.zeros(0, np.uint32)
    return np.ascontiguousarray(ids), np.ascontiguousarray(lens)


def _rows(out: np.ndarray, out_len: np.ndarray) -> list[list[int]]:
    return [out[i, : out_len[i]].tolist() for i in range(len(out_len))]


class _Ctx:
    def __init__(self, device: int):
        self.lib = load()
        h = C.c_void_p()
        check(self.lib.mlg_ctx_create(device, C.byref(h)))
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.mlg_ctx_destroy(self.h)
            self.h = None


class EncodedBatch:
    """Encoder output of one batch (cross K/V of every decoder layer, f16 in HBM)."""

    def __init__(self, lib, h, n: int):
        self.lib, self.h, self.n = lib, h, n

    def close(self):
        if getattr(self, "h", None):
            self.lib.mlg_batch_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Translator:
    """A GGUF NLLB model resident on one GPU (src/translator.rs:55-73)."""

    def __init__(self, ctx: _Ctx, handle, path: str | Path | None = None):
        self._ctx, self.lib, self.h, self.path = ctx, ctx.lib, handle, path
        c = Config()
        check(self.lib.mlg_model_config(self.h, C.byref(c)))
        self.cfg = c.as_dict()
        self._text = None

    @classmethod
    def load(cls, path: str | Path, device: int = 0) -> "Translator":
        ctx = _Ctx(device)
        h = C.c_void_p()
        check(ctx.lib.mlg_model_load(ctx.h, str(path).encode(), C.byref(h)))
        return cls(ctx, h, path)

    @property
    def text(self):
        """The model's tokenizer and text helpers (malaga_amd.text.TextCodec), read from
        the GGUF key tokenizer.huggingface.json on first use (src/translator.rs:66-68)."""
        if self._text is None:
            from .text import TextCodec

            if self.path is None:
                raise MalagaError(1, "model loaded without a path: no tokenizer")
            self._text = TextCodec.from_gguf(self.path, self.cfg)
        return self._text

    def lang_id(self, lang: str) -> int:
        """Token id of an NLLB code (``fra_Latn``) or alias (``fr``) (src/translator.rs:83-87)."""
        try:
            return self.text.lang_id(lang)
        except KeyError as e:
            raise MalagaError(1, str(e.args[0])) from None

    def translate_batch(self, texts: Sequence[str], src: str, tgt: str,
                        opts: GenOptions | None = None) -> list[str]:
        """Independent sentences in, translations out (src/translator.rs:136-167)."""
        opts = opts or GenOptions()
        self.lang_id(src), self.lang_id(tgt)  # unknown languages are errors
        return self.text.translate_batch(texts, src, tgt, lambda rows, tid, code: self.generate(
            rows, tid, dataclasses.replace(opts, shortlist=code) if opts.shortlist is True else opts))

    def translate_docs(self, docs: Sequence[str], src: str, tgt: str, opts: GenOptions | None = None) -> list[str]:
        """Documents: sentences of all documents decoded together, layout kept
        (src/translator.rs:108-133)."""
        opts = opts or GenOptions()
        self.lang_id(src), self.lang_id(tgt)
        return self.text.translate_docs(docs, src, tgt, lambda rows, tid, code: self.generate(
            rows, tid, dataclasses.replace(opts, shortlist=code) if opts.shortlist is True else opts))

    def translate(self, text: str, src: str, tgt: str, opts: GenOptions | None = None) -> str:
        """src/translator.rs:102-104."""
        return self.translate_docs([text], src, tgt, opts)[0]

    def close(self):
        if getattr(self, "h", None):
            self.lib.mlg_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def weight_bytes(self) -> int:
        return int(self.lib.mlg_model_weight_bytes(self.h))

    def budget(self, src_len: int, max_new_tokens: int | None = None) -> int:
        """Per-sentence output budget (src/translator.rs:181-182)."""
        return int(self.lib.mlg_budget(self.h, src_len, max_new_tokens or 0))

    def _out_cap(self, src, opts: GenOptions) -> int:
        return max([self.budget(len(r), opts.max_new_tokens) for r in src] + [1])

    def generate(self, src: Sequence[Sequence[int]], tgt_lang: int, opts: GenOptions | None = None) -> list[list[int]]:
        """Target ids (no specials) for tokenized sources ``[src_lang] toks [eos]``;
        sorted, batched and OOM-retried as translate_batch does (src/translator.rs:136-167)."""
        opts = opts or GenOptions()
        if not src:
            return []
        if opts.shortlist is True:  # src/translator.rs:170-172: the code is the target token
            opts = dataclasses.replace(opts, shortlist=self.text.tok.id_to_token(tgt_lang) or None)
        ids, lens = _flat(src)
        cap = self._out_cap(src, opts)
        out = np.zeros((len(src), cap), dtype=np.uint32)
        out_len = np.zeros(len(src), dtype=np.int32)
        co = opts._c()
        check(self.lib.mlg_generate(self.h, ids.ctypes.data, lens.ctypes.data, len(src), tgt_lang, C.byref(co),
                                    out.ctypes.data, cap, out_len.ctypes.data))
        return _rows(out, out_len)

    translate_batch_ids = generate

    def encode_cross(self, src: Sequence[Sequence[int]]) -> EncodedBatch:
        """Nllb::encode_cross (src/model.rs:463-477)."""
        ids, lens = _flat(src)
        h = C.c_void_p()
        check(self.lib.mlg_encode(self.h, ids.ctypes.data, lens.ctypes.data, len(src), C.byref(h)))
        return EncodedBatch(self.lib, h, len(src))

    def greedy(self, batch: EncodedBatch, tgt_lang: int, max_new: int, sync_every: int = 4,
               eos_mask: bool = False, graph: bool = True, shortlist: str | None = None) -> list[list[int]]:
        """GraphCache::greedy (src/graph.rs:204-223): rows stripped at EOS.  ``shortlist``:
        decode over that language's shortlist plus the source tokens."""
        out = np.zeros((batch.n, max_new + 1), dtype=np.uint32)
        out_len = np.zeros(batch.n, dtype=np.int32)
        flags = (FLAG_EOS_MASK if eos_mask else 0) | (0 if graph else FLAG_NO_GRAPH)
        if shortlist:
            check(self.lib.mlg_greedy_sl(self.h, batch.h, tgt_lang, shortlist.encode(), max_new, sync_every, flags,
                                         out.ctypes.data, max_new + 1, out_len.ctypes.data))
        else:
            check(self.lib.mlg_greedy(self.h, batch.h, tgt_lang, max_new, sync_every, flags, out.ctypes.data,
                                      max_new + 1, out_len.ctypes.data))
        return _rows(out, out_len)

    def greedy_top(self, batch: EncodedBatch, tgt_lang: int, max_new: int, sync_every: int = 4,
                   eos_mask: bool = False, graph: bool = True) -> tuple[list[list[int]], list[list[float]]]:
        """greedy, plus the winning logit of every returned token (parity hook of the
        fused argmax head)."""
        out = np.zeros((batch.n, max_new + 1), dtype=np.uint32)
        top = np.zeros((batch.n, max_new + 1), dtype=np.float32)
        out_len = np.zeros(batch.n, dtype=np.int32)
        flags = (FLAG_EOS_MASK if eos_mask else 0) | (0 if graph else FLAG_NO_GRAPH)
        check(self.lib.mlg_greedy_top(self.h, batch.h, tgt_lang, max_new, sync_every, flags, out.ctypes.data,
                                      top.ctypes.data, max_new + 1, out_len.ctypes.data))
        return _rows(out, out_len), [top[i, : out_len[i]].tolist() for i in range(batch.n)]

    def shortlists(self) -> dict[str, int]:
        """Languages with a vocabulary shortlist and their row counts (src/model.rs:439-447)."""
        res = {}
        for i in range(int(self.lib.mlg_model_shortlist_count(self.h))):
            code, rows = C.c_char_p(), C.c_int()
            check(self.lib.mlg_model_shortlist_info(self.h, i, C.byref(code), C.byref(rows)))
            res[code.value.decode()] = rows.value
        return res

    def beam(self, batch: EncodedBatch, tgt_lang: int, max_new: int, beam_size: int, length_penalty: float = 1.0,
             eos_mask: bool = False) -> list[list[int]]:
        """Translator::beam_search (src/translator.rs:250-335)."""
        out = np.zeros((batch.n, max_new + 1), dtype=np.uint32)
        out_len = np.zeros(batch.n, dtype=np.int32)
        check(self.lib.mlg_beam(self.h, batch.h, tgt_lang, max_new, beam_size, length_penalty,
                                FLAG_EOS_MASK if eos_mask else 0, out.ctypes.data, max_new + 1, out_len.ctypes.data))
        return _rows(out, out_len)

    def teacher_forced_logits(self, src: Sequence[Sequence[int]], tgt: np.ndarray, kv_f32: bool = False) -> np.ndarray:
        """Logits [n, T, vocab] after feeding tgt[:, t] at decoder position t; K/V in f16 (the
        graph step) or, with kv_f32, in f32 (the generic decoder, src/model.rs:514-540)."""
        ids, lens = _flat(src)
        tgt = np.ascontiguousarray(tgt, dtype=np.uint32)
        n, T = tgt.shape
        out = np.zeros((n, T, self.cfg["vocab_size"]), dtype=np.float32)
        check(self.lib.mlg_teacher_forced_logits(self.h, ids.ctypes.data, lens.ctypes.data, n, tgt.ctypes.data, T,
                                                 int(kv_f32), out.ctypes.data))
        return out

    def clear_graphs(self):
        """GraphCache::clear (src/graph.rs:192-200)."""
        self.lib.mlg_clear_graphs(self.h)

    def graph_keys(self) -> list[tuple[int, int, int, bool]]:
        """(batch, source, output) bucket and whether a graph is captured, for every cached
        state, least recently used first (src/graph.rs:301-323 evicts from the front)."""
        buf = np.zeros((64, 4), dtype=np.int32)
        n = int(self.lib.mlg_graph_cache_keys(self.h, buf.ctypes.data, 64))
        if n < 0:
            check(-n)
        return [(int(a), int(b), int(c), bool(d)) for a, b, c, d in buf[: min(n, 64)]]

    def graph_stats(self) -> dict:
        e, g, c = C.c_int(), C.c_int(), C.c_int()
        check(self.lib.mlg_graph_stats(self.h, C.byref(e), C.byref(g), C.byref(c)))
        return {"entries": e.value, "graphs": g.value, "capture": bool(c.value)}


# ----------------------------------------------------------------- configs

class Job:
    """One request queued on a Server (crates/malaga/src/server.rs:33-39)."""

    def __init__(self, server: "Server", h, n: int, cap: int):
        self.lib, self.h, self.n, self.cap, self._server = server.lib, h, n, cap, server

    def done(self, timeout_ms: int = 0) -> bool:
        d = C.c_int()
        check(self.lib.mlg_job_wait(self.h, timeout_ms, C.byref(d)))
        return bool(d.value)

    def result(self) -> list[list[int]]:
        """Blocks until the job's group has run; raises MalagaError with the group's error."""
        out = np.zeros((max(self.n, 1), self.cap), dtype=np.uint32)
        out_len = np.zeros(max(self.n, 1), dtype=np.int32)
        check(self.lib.mlg_job_result(self.h, out.ctypes.data, self.cap, out_len.ctypes.data))
        return _rows(out, out_len)[: self.n]

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.mlg_job_free(self.h)
            self.h = None


class Server:
    """Dynamic batching caller (crates/malaga/src/server.rs:74-112): a native inference
    thread decodes every queued job, grouped by (source, target, beam, shortlist), as
    one translate_batch call per group.  Submit from any number of threads."""

    def __init__(self, translator: Translator, defaults: GenOptions | None = None):
        self.t, self.lib = translator, translator.lib
        self.defaults = defaults or GenOptions()
        h = C.c_void_p()
        co = self.defaults._c()
        check(self.lib.mlg_server_start(translator.h, C.byref(co), C.byref(h)))
        self.h = h

    def submit(self, src: Sequence[Sequence[int]], tgt_lang: int, src_lang: int = 0, beam_size: int = 0,
               shortlist: str | None = None) -> Job:
        ids, lens = _flat(src)
        h = C.c_void_p()
        check(self.lib.mlg_server_submit(self.h, ids.ctypes.data, lens.ctypes.data, len(src), src_lang, tgt_lang,
                                         beam_size, shortlist.encode() if shortlist else None, C.byref(h)))
        return Job(self, h, len(src), max([self.t.budget(len(r), self.defaults.max_new_tokens) for r in src] + [1]))

    def stats(self) -> dict:
        v = [C.c_int64() for _ in range(4)]
        check(self.lib.mlg_server_stats(self.h, *[C.byref(x) for x in v]))
        return dict(zip(("jobs", "groups", "sentences", "largest_group"), (x.value for x in v)))

    def stop(self):
        if getattr(self, "h", None):
            self.lib.mlg_server_stop(self.h)
            self.h = None

    def __del__(self):
        self.stop()


def tiny_config() -> dict:
    """src/testutil.rs:18-30 (vocab 257, d 64, 4 heads, ffn 128, 2 + 2 layers)."""
    c = Config()
    load().mlg_tiny_config(C.byref(c))
    return c.as_dict()


def nllb_600m_config() -> dict:
    """NLLB-200-distilled-600M hyper-parameters."""
    return dict(vocab_size=256206, d_model=1024, encoder_layers=12, decoder_layers=12, encoder_heads=16,
                decoder_heads=16, encoder_ffn=4096, decoder_ffn=4096, max_position_embeddings=1024, max_length=200,
                scale_embedding=1, bos_token_id=0, pad_token_id=1, eos_token_id=2, decoder_start_token_id=2)


def nllb_3b_config() -> dict:
    """NLLB-200-3.3B hyper-parameters."""
    c = nllb_600m_config()
    c.update(d_model=2048, encoder_layers=24, decoder_layers=24, encoder_ffn=8192, decoder_ffn=8192)
    return c


def _cfg(d: dict) -> Config:
    c = Config()
    for k, v in d.items():
        setattr(c, k, int(v))
    return c


def _shortlist_specs(shortlists: dict | None):
    """{code: (lang_id, ids)} -> (ctypes array of ShortlistSpec, keep-alive list)."""
    from ._lib import ShortlistSpec

    items = list((shortlists or {}).items())
    arr = (ShortlistSpec * max(1, len(items)))()
    keep = []
    for i, (code, (lang_id, ids)) in enumerate(items):
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32))
        keep.append(a)
        arr[i].code = code.encode()
        arr[i].lang_id = int(lang_id)
        arr[i].ids = a.ctypes.data_as(C.POINTER(C.c_uint32))
        arr[i].n_ids = int(a.size)
    return arr, len(items), keep


def write_synthetic(path: str | Path, cfg: dict, preset: str, init: int = INIT_NORMAL, seed: int = 0,
                    std: float = 0.02, name: str = "synthetic", shortlists: dict | None = None) -> Path:
    """Random-init checkpoint converted to GGUF with the reference layout.  ``shortlists``:
    {language code: (language token id, vocabulary ids)} per-language reduced LM heads
    (src/convert.rs:218-233)."""
    lib = load()
    c = _cfg(cfg)
    arr, n, _keep = _shortlist_specs(shortlists)
    check(lib.mlg_write_synthetic_sl(str(path).encode(), C.byref(c), PRESETS[preset], init, seed, std,
                                     name.encode(), arr, n))
    return Path(path)


def convert(out_path: str | Path, cfg: dict, preset: str, tensors: Callable[[str], np.ndarray] | dict,
            model_name: str = "facebook/nllb-200-distilled-600M", tokenizer_json: str = "{}",
            shortlists: dict | None = None) -> Path:
    """src/convert.rs:196-318 from Hugging Face tensors (a dict or a name -> array function);
    ``shortlists`` as for write_synthetic."""
    lib = load()
    get = tensors.get if isinstance(tensors, dict) else tensors
    err: list[BaseException] = []

    @TENSOR_FN
    def fn(_user, name, numel, out):
        try:
            a = get(name.decode())
            if a is None:
                return 1
            a = np.ascontiguousarray(np.asarray(a, dtype=np.float32).reshape(-1))
            if a.size != numel:
                return 1
            C.memmove(out, a.ctypes.data, a.nbytes)
            return 0
        except BaseException as e:  # noqa: BLE001 - reported after the call
            err.append(e)
            return 1

    c = _cfg(cfg)
    arr, n, _keep = _shortlist_specs(shortlists)
    st = lib.mlg_convert_sl(str(out_path).encode(), C.byref(c), PRESETS[preset], model_name.encode(),
                            tokenizer_json.encode(), fn, None, arr, n)
    if err:
        raise err[0]
    check(st)
    return Path(out_path)


def convert_hf(hf_dir: str | Path, out_path: str | Path, preset: str = "q8_0", model_name: str | None = None) -> Path:
    """Converts a Hugging Face checkpoint directory (config.json + *.safetensors)."""
    from safetensors.numpy import load_file

    hf_dir = Path(hf_dir)
    hf = json.loads((hf_dir / "config.json").read_text())
    cfg = dict(vocab_size=hf["vocab_size"], d_model=hf["d_model"], encoder_layers=hf["encoder_layers"],
               decoder_layers=hf["decoder_layers"], encoder_heads=hf["encoder_attention_heads"],
               decoder_heads=hf["decoder_attention_heads"], encoder_ffn=hf["encoder_ffn_dim"],
               decoder_ffn=hf["decoder_ffn_dim"], max_position_embeddings=hf["max_position_embeddings"],
               max_length=hf.get("max_length", 200), scale_embedding=int(hf.get("scale_embedding", True)),
               bos_token_id=hf.get("bos_token_id", 0), pad_token_id=hf.get("pad_token_id", 1),
               eos_token_id=hf.get("eos_token_id", 2), decoder_start_token_id=hf.get("decoder_start_token_id", 2))
    if hf.get("activation_function", "relu") != "relu":
        raise MalagaError(6, f"unsupported activation {hf['activation_function']}")
    gen = hf_dir / "generation_config.json"
    if gen.exists():
        g = json.loads(gen.read_text())
        if "max_length" in g:
            cfg["max_length"] = g["max_length"]
    tensors: dict = {}
    for f in sorted(hf_dir.glob("*.safetensors")):
        tensors.update(load_file(str(f)))
    if "model.shared.weight" not in tensors and "model.encoder.embed_tokens.weight" in tensors:
        tensors["model.shared.weight"] = tensors["model.encoder.embed_tokens.weight"]
    tok = hf_dir / "tokenizer.json"
    return convert(out_path, cfg, preset, tensors, model_name or hf.get("_name_or_path", "nllb"),
                   tok.read_text() if tok.exists() else "{}")


# ------------------------------------------------------------------ codecs

def type_bytes(ggml_type: int, n: int) -> int:
    return int(load().mlg_type_bytes(ggml_type, n))


def quantize(ggml_type: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    nb = type_bytes(ggml_type, x.size)
    if nb < 0:
        raise MalagaError(1, "length is not a whole number of blocks")
    out = np.zeros(nb, dtype=np.uint8)
    check(load().mlg_quantize(ggml_type, x.ctypes.data, x.size, out.ctypes.data))
    return out


def dequantize(ggml_type: int, blocks: np.ndarray, n: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n, dtype=np.float32)
    check(load().mlg_dequantize(ggml_type, blocks.ctypes.data, n, out.ctypes.data))
    return out


def bucket(n: int, lo: int, hi: int) -> int:
    """src/graph.rs:138-140."""
    return int(load().mlg_bucket(n, lo, hi))
