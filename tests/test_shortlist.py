"""Vocabulary shortlists (--fast-vocab): the GGUF layout written by the converter and the
oracle's restricted greedy (src/convert.rs:176-233, src/model.rs:594-603,
kernels/malaga.cu:229-326).  CPU only."""
import numpy as np
import pytest

import malaga_amd as M
import oracle as O
from malaga_amd.gguf import read_gguf, tensor_bytes

FRA = 254  # language token of the tiny vocabulary (src/testutil.rs:33-54)


@pytest.fixture(scope="module")
def sl_gguf(tmp_path_factory):
    d = tmp_path_factory.mktemp("sl")

    def make(preset: str, ids):
        p = d / f"tiny-sl-{preset}-{len(ids)}.gguf"
        if not p.exists():
            M.write_synthetic(p, M.tiny_config(), preset, M.INIT_TESTUTIL, seed=7, name="tiny",
                              shortlists={"fra_Latn": (FRA, ids)})
        return p

    return make


@pytest.mark.parametrize("preset", ["f32", "q8_0"])
def test_writer_stores_token_embd_rows_and_sorted_ids(sl_gguf, preset):
    ids = [200, 17, 17, 9999, 5, 42]
    p = sl_gguf(preset, ids)
    _, meta, tensors, _ = read_gguf(p)
    got = meta["nllb.shortlist.fra_Latn"]
    want = sorted({0, 1, 2, 3, FRA, 200, 17, 5, 42})  # ids >= vocab dropped, specials and language added
    assert got == want
    emb, ei = tensor_bytes(p, "token_embd.weight")
    head, hi = tensor_bytes(p, "lm_head.fra_Latn.weight")
    assert hi["type"] == ei["type"] and hi["ne"] == [ei["ne"][0], len(want)]
    rb = emb.size // ei["ne"][1]
    for r, t in enumerate(want):
        assert bytes(head[r * rb:(r + 1) * rb]) == bytes(emb[t * rb:(t + 1) * rb])


def test_oracle_full_shortlist_equals_full_vocabulary(sl_gguf):
    p = sl_gguf("q8_0", list(range(257)))
    m = O.Model(p)
    src = [[FRA, 5, 6, 7, 8, 2], [FRA, 40, 41, 2]]
    full, _ = m.generate(src, FRA, max_new_tokens=10)
    short, _ = m.generate(src, FRA, max_new_tokens=10, shortlist=list(range(257)))
    assert full == short


def _stepwise(m, src_row, tgt, shortlist, max_new, eos):
    """Independent restatement on the oracle's logits: teacher-force the tokens chosen so
    far and take the argmax over [shortlist..., source tokens...] (first maximum)."""
    toks = [2, tgt]
    for _ in range(max_new):
        lg = m.teacher_forced_logits([src_row], np.array([toks], dtype=np.uint32), kv_f16=False)[0, -1]
        cand = list(shortlist) + list(src_row)
        vals = [lg[t] for t in cand]
        t = cand[int(np.argmax(vals))]
        toks.append(t)
        if t == eos:
            break
    out = toks[2:]
    return out[: out.index(eos)] if eos in out else out


SL_IDS = sorted(set(np.random.default_rng(3).integers(4, 1000, 300).tolist()) - {76, 258, 607, 884, 738, 182, 267, 931})


def shortlist_fixture(path, preset):
    """d = 256 model whose greedy output varies (unscaled embeddings, std 0.2), with a
    shortlist that leaves out the tokens the full model prefers: those can then only be
    produced as copies of source tokens.  A second shortlist, "eng_Latn" (language id
    997), lacks token 998 and so cannot serve decoding into 998."""
    from conftest import KQ_CONFIG

    if not path.exists():
        M.write_synthetic(path, dict(KQ_CONFIG, scale_embedding=0), preset, M.INIT_NORMAL_RICH, seed=11, std=0.2,
                          name="kq-sl", shortlists={"fra_Latn": (998, SL_IDS),
                                                    "eng_Latn": (997, [t for t in SL_IDS if t != 998])})
    return path, read_gguf(path)[1]["nllb.shortlist.fra_Latn"]


SL_SOURCES = [[997, 76, 6, 7, 8, 2], [997, 100, 607, 102, 2], [997, 9, 258, 2], [997, 182, 267, 2]]


def test_oracle_shortlist_matches_stepwise_restatement(tmp_path):
    p, sl = shortlist_fixture(tmp_path / "kq-sl-f32.gguf", "f32")
    m = O.Model(p)
    got, gap = m.generate(SL_SOURCES, 998, max_new_tokens=8, shortlist=sl, kv_f16=False)
    assert gap > 1e-3
    copies = 0
    for s, g in zip(SL_SOURCES, got):
        assert g == _stepwise(m, s, 998, sl, 8, 2)
        assert all(t in sl or t in s for t in g)
        copies += sum(t not in sl for t in g)
    assert copies > 0  # the source candidates are exercised
