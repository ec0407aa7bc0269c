"""Host text path around the decoder: sentence segmentation, language codes, the
tokenizer, and documents in / documents out.

* ``segment`` restates src/segment.rs:24-99 with Rust ``char`` semantics:
  ``is_whitespace`` = Unicode White_Space, ``is_uppercase`` = the Uppercase derived
  property (CPython's ``str.isupper`` on one character), ``is_numeric`` = general
  category N*.  Unicode tables are Python's (``unicodedata.unidata_version``).
* ``resolve`` restates src/langs.rs:10-21.
* The tokenizer is Hugging Face ``tokenizers`` 0.22.2, the version the reference
  pins (Cargo.lock), read from the GGUF key ``tokenizer.huggingface.json``
  (src/translator.rs:66-68).
* ``TextCodec`` holds the tokenizer and the model's special ids: ``encode`` is
  src/translator.rs:90-98, ``translate_batch`` / ``translate_docs`` are
  src/translator.rs:108-167 with a pluggable batch decoder (the GPU Translator, or
  the CPU oracle in tests).
"""
from __future__ import annotations

import unicodedata
from collections import Counter
from pathlib import Path
from typing import Callable, Iterable, Sequence

# Unicode White_Space (char::is_whitespace; str::trim trims these)
_WHITE_SPACE = frozenset([chr(c) for c in range(0x09, 0x0E)] + [chr(c) for c in range(0x2000, 0x200B)] + [
    " ", "\x85", "\xa0", "\u1680", "\u2028", "\u2029", "\u202f", "\u205f", "\u3000"])

# src/segment.rs:12-15
ABBREVIATIONS = ("M", "Mme", "Mlle", "Dr", "Pr", "St", "Ste", "Mr", "Mrs", "Ms", "Prof", "etc", "cf", "p", "n", "vol",
                 "ex", "e.g", "i.e", "vs", "Jr", "Sr", "No", "art")

_ENDERS = ".!?…。"
_TRAILERS = ".!?\"»”')’"
_CLOSERS = "»”"
_STARTERS = "\"«“(-—"


def _ws(c: str) -> bool:
    return c in _WHITE_SPACE


def _upper(c: str) -> bool:
    return c.isupper()


def _numeric(c: str) -> bool:
    return unicodedata.category(c)[0] == "N"


def _trim_start(s: str) -> str:
    i = 0
    while i < len(s) and _ws(s[i]):
        i += 1
    return s[i:]


def _trim(s: str) -> str:
    s = _trim_start(s)
    j = len(s)
    while j > 0 and _ws(s[j - 1]):
        j -= 1
    return s[:j]


def _ascii_lower(s: str) -> str:
    return "".join(chr(ord(c) + 32) if "A" <= c <= "Z" else c for c in s)


def is_abbreviation(before: str) -> bool:
    """src/segment.rs:17-22: the word before a period is a known abbreviation (ASCII
    case-insensitive) or a single uppercase letter."""
    k = len(before)
    while k > 0 and not (_ws(before[k - 1]) or before[k - 1] == "("):
        k -= 1
    word = before[k:].rstrip(".")
    lw = _ascii_lower(word)
    return any(_ascii_lower(a) == lw for a in ABBREVIATIONS) or (len(word) == 1 and _upper(word))


def _split_line(line: str, out: list) -> None:
    """src/segment.rs:35-99."""
    body = _trim(line)
    if not body:
        if line:
            out.append((False, line))
        return
    lead = len(line) - len(_trim_start(line))
    if lead:
        out.append((False, line[:lead]))
    n = len(body)

    def skip_ws(k: int) -> int:
        while k < n and _ws(body[k]):
            k += 1
        return k

    start = i = 0
    while i < n:
        c = body[i]
        if c in _ENDERS:
            # trailing punctuation / closing quotes belong to the sentence
            j = i + 1
            while True:
                if j < n and body[j] in _TRAILERS:
                    j += 1
                elif skip_ws(j) < n and body[skip_ws(j)] in _CLOSERS:  # French spacing: « oui. »
                    j = skip_ws(j) + 1
                else:
                    break
            ws_end = skip_ws(j)
            followed = ws_end > j and ws_end < n and (
                _upper(body[ws_end]) or _numeric(body[ws_end]) or body[ws_end] in _STARTERS)
            if followed and not (c == "." and is_abbreviation(body[start:i])):
                end = min(j, n)
                out.append((True, body[start:end]))
                out.append((False, body[end:ws_end]))
                start = i = ws_end
                continue
            i = j
            continue
        i += 1
    out.append((True, body[start:]))
    tail = line[lead + len(body):]
    if tail:
        out.append((False, tail))


def segment(text: str) -> list[tuple[bool, str]]:
    """src/segment.rs:24-33: (is_sentence, piece) in order; the pieces concatenate back
    to ``text``.  Lines are split on '\\n' only."""
    out: list = []
    for i, line in enumerate(text.split("\n")):
        if i > 0:
            out.append((False, "\n"))
        _split_line(line, out)
    return out


def resolve(lang: str) -> str:
    """src/langs.rs:10-21: aliases of fr / en / mg to NLLB codes; anything else as is."""
    s = _trim(lang)
    lower = s.lower()
    base = lower.replace("_", "-").split("-")[0]
    if base in ("fr", "fra", "fre", "french", "français", "francais"):
        return "fra_Latn"
    if base in ("en", "eng", "english", "anglais"):
        return "eng_Latn"
    if base in ("mg", "mlg", "plt", "malagasy", "malgache"):
        return "plt_Latn"
    return s


def load_tokenizer(tokenizer_json: str):
    from tokenizers import Tokenizer

    return Tokenizer.from_str(tokenizer_json)


def gguf_tokenizer_json(path: str | Path) -> str:
    from .gguf import read_gguf

    meta = read_gguf(path)[1]
    tj = meta.get("tokenizer.huggingface.json")
    if not tj:
        raise ValueError(f"{path}: no tokenizer.huggingface.json in the GGUF metadata")
    return tj


def shortlist_ids(tokenizer, lines: Iterable[str], min_count: int, vocab: int) -> list[int]:
    """src/convert.rs:174-193: ids seen at least ``min_count`` times when tokenizing the
    non-blank corpus lines (no special tokens added), plus ids 0..3.  Sorted."""
    counts: Counter = Counter()
    batch = [ln for ln in lines if _trim(ln)]
    for k in range(0, len(batch), 4096):
        for enc in tokenizer.encode_batch(batch[k:k + 4096], add_special_tokens=False):
            counts.update(enc.ids)
    return [i for i in range(vocab) if i < 4 or counts.get(i, 0) >= min_count]


def corpus_shortlist(tokenizer_json: str, lang: str, corpus: str | Path, vocab: int,
                     min_count: int = 2) -> tuple[str, tuple[int, list[int]]]:
    """``convert --shortlist LANG=corpus`` (src/convert.rs:215-233, min count default 2 as
    crates/malaga/src/main.rs:43-45): (code, (language id, ids)) for the converter's
    ``shortlists`` argument, which adds the language id."""
    tok = load_tokenizer(tokenizer_json)
    code = resolve(lang)
    lang_id = tok.token_to_id(code)
    if lang_id is None:
        raise ValueError(f"unknown language {lang}")
    # str::lines: split at "\n", a trailing "\r" dropped
    lines = [ln[:-1] if ln.endswith("\r") else ln for ln in Path(corpus).read_text(encoding="utf-8").split("\n")]
    return code, (lang_id, shortlist_ids(tok, lines, min_count, vocab))


class TextCodec:
    """Tokenizer + special ids of one model: text <-> source / target ids."""

    def __init__(self, tokenizer_json: str, cfg: dict):
        self.tok = load_tokenizer(tokenizer_json)
        self.cfg = cfg

    @classmethod
    def from_gguf(cls, path: str | Path, cfg: dict) -> "TextCodec":
        return cls(gguf_tokenizer_json(path), cfg)

    def lang_id(self, lang: str) -> int:
        """src/translator.rs:83-87."""
        code = resolve(lang)
        i = self.tok.token_to_id(code)
        if i is None:
            raise KeyError(f"unknown language '{lang}' (NLLB code '{code}')")
        return i

    def encode(self, text: str, src_id: int) -> list[int]:
        """src/translator.rs:90-98: [src_lang] tokens [eos], tokens cut at max_pos - 2."""
        ids = self.tok.encode(text, add_special_tokens=False).ids
        return [src_id] + ids[: self.cfg["max_position_embeddings"] - 2] + [self.cfg["eos_token_id"]]

    def decode(self, ids: Sequence[int]) -> str:
        return self.tok.decode(list(ids), skip_special_tokens=True)

    def translate_batch(self, texts: Sequence[str], src: str, tgt: str,
                        generate: Callable[[list, int, str], list]) -> list[str]:
        """src/translator.rs:136-167 above ``generate(ids_rows, tgt_id, tgt_code)``, which
        sorts, batches and retries as translate_batch does on ids."""
        tgt_code = resolve(tgt)
        sid, tid = self.lang_id(src), self.lang_id(tgt)
        rows = generate([self.encode(t, sid) for t in texts], tid, tgt_code)
        return [self.decode(r) for r in rows]

    def translate_docs(self, docs: Sequence[str], src: str, tgt: str,
                       generate: Callable[[list, int, str], list]) -> list[str]:
        """src/translator.rs:108-133: every sentence of every document in one
        translate_batch call; separators (newlines, spaces) kept as they were."""
        segs = [segment(d) for d in docs]
        texts = [t for s in segs for is_text, t in s if is_text]
        it = iter(self.translate_batch(texts, src, tgt, generate) if texts else [])
        return ["".join(next(it) if is_text else t for is_text, t in s) for s in segs]
