"""Shortlist (--fast-vocab) greedy decoding on the GPU against the oracle's restricted
greedy: candidates are the shortlist rows then the source tokens, the next input
embedding comes from the shortlist head or the copied source position
(src/model.rs:552-612, src/graph.rs:40-130, kernels/malaga.cu:108-118, 229-243, 283-326).
Tokens bit-exact."""
import numpy as np
import pytest

import malaga_amd as M
from malaga_amd import MalagaError
import oracle as O
from tests.test_shortlist import SL_SOURCES, shortlist_fixture

pytestmark = pytest.mark.gpu
FRA, ENG = 998, 997


@pytest.fixture(scope="module")
def sl_models(model_dir):
    cache = {}

    def get(preset):
        if preset not in cache:
            p, sl = shortlist_fixture(model_dir / f"kq-sl-{preset}.gguf", preset)
            cache[preset] = (M.Translator.load(p), O.Model(p), sl)
        return cache[preset]

    return get


def _sources(nb, seed):
    rng = np.random.default_rng(seed)
    extra = [[ENG] + rng.integers(4, 990, int(n)).tolist() + [2] for n in rng.integers(2, 30, max(0, nb - 4))]
    return (SL_SOURCES + extra)[:nb]


@pytest.mark.parametrize("preset", ["f32", "q8_0", "q4_k_m", "q5_k_m"])
@pytest.mark.parametrize("nb", [1, 2, 4, 7, 16])
def test_shortlist_greedy_matches_oracle(sl_models, preset, nb):
    """nb <= 4: fused step kernels; larger batches: the MFMA step with the batched head."""
    gpu, orc, sl = sl_models(preset)
    src = _sources(nb, 40 + nb)
    want, gap = orc.translate_batch(src, FRA, kv_f16=True, max_new_tokens=12, shortlist=sl)
    got = gpu.generate(src, FRA, M.GenOptions(max_new_tokens=12, shortlist="fra_Latn"))
    assert got == want, f"min top-2 gap {gap}"
    slset = set(sl)
    for s, g in zip(src, got):
        assert all(t in slset or t in s for t in g)


def test_shortlist_copies_source_tokens(sl_models):
    """The fixture's full model prefers tokens outside the shortlist; they can only come
    from the source candidates, and the next step then embeds the copied position."""
    gpu, orc, sl = sl_models("f32")
    got = gpu.generate(SL_SOURCES, FRA, M.GenOptions(max_new_tokens=12, shortlist="fra_Latn"))
    want, _ = orc.translate_batch(SL_SOURCES, FRA, kv_f16=True, max_new_tokens=12, shortlist=sl)
    assert got == want
    slset = set(sl)
    assert sum(t not in slset for g in got for t in g) > 0


@pytest.mark.parametrize("graph", [True, False])
def test_shortlist_boundary_entry_point(sl_models, graph):
    """mlg_greedy_sl on an encoded batch, with the step graph and eagerly; the graph
    cache keys on the shortlist, so exact and shortlist decoding of the same shapes
    alternate without mixing."""
    gpu, orc, sl = sl_models("q8_0")
    b = gpu.encode_cross(SL_SOURCES)
    want_sl, _ = orc.generate(SL_SOURCES, FRA, kv_f16=True, max_new_tokens=10, shortlist=sl)
    want_full, _ = orc.generate(SL_SOURCES, FRA, kv_f16=True, max_new_tokens=10)
    for _ in range(2):
        assert gpu.greedy(b, FRA, 10, graph=graph, shortlist="fra_Latn") == want_sl
        assert gpu.greedy(b, FRA, 10, graph=graph) == want_full


def test_shortlist_eos_mask_fixed_lengths(sl_models):
    gpu, orc, sl = sl_models("q4_k_m")
    want, _ = orc.translate_batch(SL_SOURCES, FRA, kv_f16=True, max_new_tokens=9, shortlist=sl, eos_mask=True)
    got = gpu.generate(SL_SOURCES, FRA, M.GenOptions(max_new_tokens=9, shortlist="fra_Latn", eos_mask=True))
    assert got == want and all(len(g) == 9 for g in got)


def test_shortlist_selection_rules(sl_models):
    """src/translator.rs:184-194: a shortlist without the target language, beam search and
    the unfused option all decode exactly; an unknown code is an error at the boundary."""
    gpu, orc, sl = sl_models("q8_0")
    lists = gpu.shortlists()
    assert set(lists) == {"fra_Latn", "eng_Latn"} and lists["fra_Latn"] == len(sl)
    exact, _ = orc.translate_batch(SL_SOURCES, FRA, kv_f16=True, max_new_tokens=8)
    assert gpu.generate(SL_SOURCES, FRA, M.GenOptions(max_new_tokens=8, shortlist="eng_Latn")) == exact
    assert gpu.generate(SL_SOURCES, FRA, M.GenOptions(max_new_tokens=8, shortlist="xxx_Latn")) == exact
    beam, _ = orc.translate_batch(SL_SOURCES, FRA, kv_f16=True, max_new_tokens=8, beam_size=2)
    assert gpu.generate(SL_SOURCES, FRA, M.GenOptions(max_new_tokens=8, beam_size=2, shortlist="fra_Latn")) == beam
    b = gpu.encode_cross(SL_SOURCES[:1])
    with pytest.raises(MalagaError):
        gpu.greedy(b, FRA, 4, shortlist="xxx_Latn")
    with pytest.raises(MalagaError):  # token 998 missing from the eng_Latn shortlist
        gpu.greedy(b, FRA, 4, shortlist="eng_Latn")


def test_lazy_embeddings(sl_models, model_dir, monkeypatch):
    """MALAGA_LAZY_EMBEDDINGS (src/model.rs:252-307, 416-420): token_embd stays on the host
    while shortlist decoding runs (encoder and source rows gathered from the host copy)
    and is uploaded once when exact decoding needs the full LM head."""
    from malaga_amd.gguf import tensor_bytes

    eager, orc, sl = sl_models("q4_k_m")
    p = model_dir / "kq-sl-q4_k_m.gguf"
    monkeypatch.setenv("MALAGA_LAZY_EMBEDDINGS", "1")
    lazy = M.Translator.load(p)
    monkeypatch.delenv("MALAGA_LAZY_EMBEDDINGS")
    raw, info = tensor_bytes(p, "token_embd.weight")
    # the resident table, plus the lane-major quant copy a q6_K LM head carries (192 B per
    # block) and the tile-major copy of a q6_K / q4_K one (3456 / 2304 B per 16-row tile and
    # 256-wide block)
    emb_bytes = raw.size
    K, V = info["ne"][0], info["ne"][1]
    if info["type"] == 14:
        emb_bytes += raw.size // 210 * 192 + (V + 15) // 16 * (K // 256) * 3456
    elif info["type"] == 12:
        emb_bytes += (V + 15) // 16 * (K // 256) * 2304
    assert lazy.weight_bytes == eager.weight_bytes - emb_bytes
    for nb in (4, 7):
        src = _sources(nb, 70 + nb)
        want, _ = orc.translate_batch(src, FRA, kv_f16=True, max_new_tokens=10, shortlist=sl)
        assert lazy.generate(src, FRA, M.GenOptions(max_new_tokens=10, shortlist="fra_Latn")) == want
    assert lazy.weight_bytes == eager.weight_bytes - emb_bytes
    exact, _ = orc.translate_batch(SL_SOURCES, FRA, kv_f16=True, max_new_tokens=10)
    assert lazy.generate(SL_SOURCES, FRA, M.GenOptions(max_new_tokens=10)) == exact
    assert lazy.weight_bytes == eager.weight_bytes
    want, _ = orc.translate_batch(SL_SOURCES, FRA, kv_f16=True, max_new_tokens=10, shortlist=sl)
    assert lazy.generate(SL_SOURCES, FRA, M.GenOptions(max_new_tokens=10, shortlist="fra_Latn")) == want
    lazy.close()
