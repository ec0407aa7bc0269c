"""Host text path (CPU): segmentation (src/segment.rs), language codes (src/langs.rs),
the tokenizer round trip and documents through a batch decoder (src/translator.rs:
90-167), corpus shortlists (src/convert.rs:174-233).  The decoder here is the CPU
oracle; the GPU tests run the same path on the HIP library."""
import pytest

import malaga_amd as M
import oracle as O
from malaga_amd.gguf import read_gguf
from malaga_amd.text import TextCodec, corpus_shortlist, gguf_tokenizer_json, resolve, segment


def texts(s):
    return [t for is_text, t in segment(s) if is_text]


def rebuild(s):
    return "".join(t for _, t in segment(s))


def test_reference_sentences():
    """src/segment.rs:118-127."""
    assert texts("Bonjour M. Dupont. Comment allez-vous ? Très bien !") == [
        "Bonjour M. Dupont.", "Comment allez-vous ?", "Très bien !"]
    assert texts("Hello world") == ["Hello world"]
    assert texts("Version 2.5 is out. Great.") == ["Version 2.5 is out.", "Great."]
    assert texts("Il a dit « oui. » Puis il est parti.") == ["Il a dit « oui. »", "Puis il est parti."]


@pytest.mark.parametrize("s", ["A. B.\n\n  C!  \nD", "", "\n", "x\n", "  lead", "Un. Deux.   Trois.",
                               "A.\r\nB.", "Oui.\u00a0Non.", "\u3000x\u3000", "\u2026", "a.\n\n\nb"])
def test_layout_is_preserved(s):
    """src/segment.rs:130-135 (first six cases) and more: pieces concatenate back."""
    assert rebuild(s) == s


@pytest.mark.parametrize("s, want", [
    ("Dr. Smith arrived. He left.", ["Dr. Smith arrived.", "He left."]),           # listed abbreviation
    ("J. R. R. Tolkien wrote. Yes.", ["J. R. R. Tolkien wrote.", "Yes."]),         # single capital
    ("It costs 5 €. 30 people came.", ["It costs 5 €.", "30 people came."]),       # numeric start
    ("Wait... What?", ["Wait...", "What?"]),                                       # trailing periods
    ('He said "stop." Then left.', ['He said "stop."', "Then left."]),             # closing quote
    ("end. lower case continues", ["end. lower case continues"]),                  # no capital after
    ("Hi!Next", ["Hi!Next"]),                                                      # no whitespace
    ("a\u3002 B", ["a\u3002", "B"]),                                               # ideographic stop
    ("See p. 5 now. Ok", ["See p. 5 now.", "Ok"]),                                 # 'p' abbreviation
    ("Call No. 5. Done", ["Call No. 5.", "Done"]),
    ("(etc. Fine", ["(etc. Fine"]),                                                # '(' ends the word
    ("ETC. Fine", ["ETC. Fine"]),                                                  # ASCII case-insensitive
    ("É. Fine", ["É. Fine"]),                                                      # one capital, non-ASCII
    ("Oui.\u00a0Non.", ["Oui.", "Non."]),                                          # NBSP is White_Space
    ("Oui.\u200bNon.", ["Oui.\u200bNon."]),                                        # ZWSP is not
    ("Go! « Now »", ["Go!", "« Now »"]),                                           # opening guillemet
    ("A.\r\nB.", ["A.", "B."]),
])
def test_segment_rules(s, want):
    assert texts(s) == want
    assert rebuild(s) == s


def test_separators():
    assert segment("Un. Deux.   Trois.") == [(True, "Un."), (False, " "), (True, "Deux."), (False, "   "),
                                             (True, "Trois.")]
    assert segment("  a\n") == [(False, "  "), (True, "a"), (False, "\n")]
    assert segment("A.\r\nB.") == [(True, "A."), (False, "\r"), (False, "\n"), (True, "B.")]


def test_language_aliases():
    """src/langs.rs:27-38."""
    for a, code in [("fr", "fra_Latn"), ("fr-FR", "fra_Latn"), ("Français", "fra_Latn"), ("en_US", "eng_Latn"),
                    ("MG", "plt_Latn"), ("malgache", "plt_Latn"), ("plt_Latn", "plt_Latn"), ("deu_Latn", "deu_Latn"),
                    (" english ", "eng_Latn")]:
        assert resolve(a) == code


@pytest.fixture(scope="module")
def tiny_codec(tiny_gguf):
    p = tiny_gguf("f32")
    return p, TextCodec.from_gguf(p, M.tiny_config())


def test_tokenizer_round_trip(tiny_codec):
    _, t = tiny_codec
    assert [t.lang_id(x) for x in ("fr", "en", "mg")] == [254, 255, 256]
    assert t.encode("w1 w2 w3", 254) == [254, 5, 6, 7, 2]
    assert t.encode("w1 zzz", 254) == [254, 5, 3, 2]  # unknown word -> <unk>
    assert t.decode([5, 6, 7, 2, 256]) == "w1 w2 w3"    # specials skipped
    with pytest.raises(KeyError):
        t.lang_id("klingon")
    long = " ".join(["w1"] * 300)
    assert len(t.encode(long, 254)) == M.tiny_config()["max_position_embeddings"]


def test_documents_through_the_oracle(tiny_codec):
    """pipeline.rs:74-81 (document layout) and pipeline.rs:30-42 (non-empty output),
    with the CPU oracle as the batch decoder."""
    p, t = tiny_codec
    orc = O.Model(p)
    dec = lambda rows, tid, code: orc.translate_batch(rows, tid, kv_f16=False)[0]  # noqa: E731
    out = t.translate_docs(["w1 w2.\n\n  w3 w4!\nw5"], "fr", "mg", dec)[0]
    assert out.count("\n") == 3 and "\n\n  " in out
    one = t.translate_batch(["w1 w2 w3. w4 w5"], "fr", "mg", dec)
    assert one[0] != ""
    # sentences of several documents share the batches; each keeps its own layout
    docs = ["w1 w2. W3 w4", "w5\nw6 w7"]
    got = t.translate_docs(docs, "fr", "mg", dec)
    assert got == [t.translate_docs([d], "fr", "mg", dec)[0] for d in docs]


def test_corpus_shortlist(tmp_path, tiny_gguf):
    """pipeline.rs:83-96: tokens seen in the corpus (min count 1), the specials and the
    language token are kept; unseen tokens are not."""
    tj = gguf_tokenizer_json(tiny_gguf("f32"))
    corpus = tmp_path / "mg.txt"
    corpus.write_text("w1 w2 w3\nw2 w9\n")
    code, (lang, ids) = corpus_shortlist(tj, "mg", corpus, M.tiny_config()["vocab_size"], min_count=1)
    assert code == "plt_Latn" and lang == 256
    p = tmp_path / "tiny-sl.gguf"
    M.write_synthetic(p, M.tiny_config(), "q8_0", M.INIT_TESTUTIL, seed=7, name="tiny", shortlists={code: (lang, ids)})
    sl = read_gguf(p)[1]["nllb.shortlist.plt_Latn"]
    for i in (0, 1, 2, 3, 5, 6, 7, 13, 256):
        assert i in sl
    assert 4 + 100 not in sl
    _, (_, ids2) = corpus_shortlist(tj, "mg", corpus, M.tiny_config()["vocab_size"])  # default min count 2
    assert ids2 == [0, 1, 2, 3, 6]  # only w2 is seen twice
