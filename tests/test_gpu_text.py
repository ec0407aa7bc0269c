"""Text in, text out on the GPU: crates/malaga-core/tests/pipeline.rs on the HIP
library (every preset translates; batching does not change translations; beam 1 is
greedy; document layout; unknown languages; fused == eager; --fast-vocab from a corpus
shortlist), each checked against the same text path with the CPU oracle decoding."""
import pytest

import malaga_amd as M
from malaga_amd import MalagaError
import oracle as O
from malaga_amd.gguf import read_gguf
from malaga_amd.text import TextCodec, corpus_shortlist, gguf_tokenizer_json

pytestmark = pytest.mark.gpu


def sentences():
    """src/testutil.rs:103-106 sentence(3 + 4i, i) as text."""
    return [" ".join(f"w{(i * 31 + k * 17) % 250}" for k in range(3 + 4 * i)) for i in range(6)]


def oracle_docs(p, docs, **kw):
    orc = O.Model(p)
    dec = lambda rows, tid, code: orc.translate_batch(rows, tid, kv_f16=True, **kw)[0]  # noqa: E731
    return TextCodec.from_gguf(p, M.tiny_config()).translate_docs(docs, "fr", "mg", dec)


@pytest.mark.parametrize("preset", ["f32", "f16", "q8_0", "q4_k_m"])
def test_every_preset_translates(tiny_gguf, preset):
    p = tiny_gguf(preset)
    T = M.Translator.load(p)
    out = T.translate("w1 w2 w3. w4 w5", "fr", "mg")
    assert out and out == oracle_docs(p, ["w1 w2 w3. w4 w5"])[0]
    T.close()


def test_batching_and_fused_paths(tiny_gguf):
    p = tiny_gguf("f32")
    T = M.Translator.load(p)
    s = sentences()
    batched = T.translate_batch(s, "fr", "mg")
    assert batched == [T.translate_batch([x], "fr", "mg")[0] for x in s]
    assert batched == T.translate_batch(s, "fr", "mg", M.GenOptions(fused=False))
    assert batched == oracle_docs(p, s)
    one = sentences()[2]
    assert T.translate(one, "fr", "mg", M.GenOptions(beam_size=1)) == T.translate(one, "fr", "mg")
    b3 = T.translate(one, "fr", "mg", M.GenOptions(beam_size=3))
    assert b3 == T.translate(one, "fr", "mg", M.GenOptions(beam_size=3))
    T.close()


def test_document_layout_and_languages(tiny_gguf):
    p = tiny_gguf("q8_0")
    T = M.Translator.load(p)
    doc = "w1 w2.\n\n  w3 w4!\nw5"
    out = T.translate(doc, "fr", "mg")
    assert out.count("\n") == 3 and "\n\n  " in out
    assert out == oracle_docs(p, [doc])[0]
    with pytest.raises(MalagaError):
        T.translate("w1", "fr", "klingon")
    assert T.lang_id("français") == 254
    T.close()


def test_fast_vocab_from_a_corpus_shortlist(tiny_gguf, tmp_path):
    src = tiny_gguf("q8_0")
    corpus = tmp_path / "mg.txt"
    corpus.write_text("\n".join(sentences()) + "\nw1 w2 w3\n")
    code, (lang, ids) = corpus_shortlist(gguf_tokenizer_json(src), "mg", corpus, M.tiny_config()["vocab_size"],
                                         min_count=1)
    p = tmp_path / "tiny-sl.gguf"
    M.write_synthetic(p, M.tiny_config(), "q8_0", M.INIT_TESTUTIL, seed=7, name="tiny", shortlists={code: (lang, ids)})
    T = M.Translator.load(p)
    docs = ["w1 w2 w3. w4 w5", sentences()[3]]
    got = T.translate_docs(docs, "fr", "mg", M.GenOptions(shortlist=True))
    assert got == oracle_docs(p, docs, shortlist=read_gguf(p)[1]["nllb.shortlist.plt_Latn"])
    T.close()
