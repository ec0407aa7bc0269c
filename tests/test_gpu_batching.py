"""The batching policy around the decoder on the GPU: the graph cache's LRU budget
(src/graph.rs:149-150, 182-186, 243-255, 301-323) and translate_batch's chunking and
out-of-memory halving (src/translator.rs:136-167), forced from the host.  Tokens always
equal the oracle's (f16 K/V emulated).
"""
import os

import pytest

import malaga_amd as M
import oracle as O
from malaga_amd import _lib
from tests.conftest import pipeline_sentences

pytestmark = pytest.mark.gpu
PLT = 256  # plt_Latn in the tiny vocabulary
MAX_NEW = 12  # fixed output budget: one output bucket (m = 32) for every call


def load_with_env(path, **env):
    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return M.Translator.load(path)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.fixture(scope="module")
def tiny(tiny_gguf):
    path = tiny_gguf("q8_0")
    return path, O.Model(path)


def oracle_rows(orc, src, max_batch=32):
    return orc.translate_batch(src, PLT, max_batch=max_batch, max_new_tokens=MAX_NEW, kv_f16=True)[0]


def opts(**kw):
    return M.GenOptions(max_new_tokens=MAX_NEW, **kw)


def test_lru_keeps_the_recently_used_bucket(tiny):
    """A 72 MB budget holds two captured graphs (32 MB each, src/graph.rs:150, plus the
    tiny states): inserting a third state (+ the 32 MB reserve for its graph) evicts the
    least recently used one, never the entry being inserted."""
    path, orc = tiny
    gpu = load_with_env(path, MALAGA_GRAPH_CACHE_MB=72)
    src = pipeline_sentences()
    try:
        one, two, three = src[:1], src[1:3], src[3:6]
        for batch in (one, two, one):  # buckets b = 1, 2, then 1 again (now the most recent)
            assert gpu.generate(batch, PLT, opts()) == oracle_rows(orc, batch)
        assert [k[0] for k in gpu.graph_keys()] == [2, 1]
        assert all(k[3] for k in gpu.graph_keys())
        assert gpu.generate(three, PLT, opts()) == oracle_rows(orc, three)  # bucket b = 4
        keys = gpu.graph_keys()
        assert [k[0] for k in keys] == [1, 4], keys  # b = 2 was least recently used
        assert all(k[3] for k in keys)
        # the evicted bucket comes back as a fresh state and graph, same tokens
        assert gpu.generate(two, PLT, opts()) == oracle_rows(orc, two)
        assert [k[0] for k in gpu.graph_keys()] == [4, 2]
    finally:
        gpu.close()


@pytest.mark.parametrize("mb", [0, 40])
def test_budget_below_two_graphs_keeps_only_the_current_entry(tiny, mb):
    """MALAGA_GRAPH_CACHE_MB=0 (any budget under two graphs) leaves one entry: the one in
    use (the eviction loop stops at one entry, src/graph.rs:306)."""
    path, orc = tiny
    gpu = load_with_env(path, MALAGA_GRAPH_CACHE_MB=mb)
    src = pipeline_sentences()
    try:
        for batch in (src[:1], src[1:3], src[3:6], src[:1]):
            assert gpu.generate(batch, PLT, opts()) == oracle_rows(orc, batch)
            assert len(gpu.graph_keys()) == 1
            assert gpu.graph_keys()[0][0] == {1: 1, 2: 2, 3: 4}[len(batch)]
    finally:
        gpu.close()


@pytest.mark.parametrize("value", ["99999999999999999999999", "18446744073709551616", "12x", "-5", ""])
def test_budget_parse_error_means_512_mb(tiny, value):
    """src/graph.rs:183: a value Rust's str::parse::<usize> rejects (more than 64 bits, a
    sign, other characters, empty) falls back to 512 MB, which keeps all three tiny
    states here; an overflowing number must not wrap to a small budget."""
    path, orc = tiny
    gpu = load_with_env(path, MALAGA_GRAPH_CACHE_MB=value)
    src = pipeline_sentences()
    try:
        for batch in (src[:1], src[1:3], src[3:6]):
            assert gpu.generate(batch, PLT, opts()) == oracle_rows(orc, batch)
        assert sorted(k[0] for k in gpu.graph_keys()) == [1, 2, 4]
    finally:
        gpu.close()


@pytest.mark.parametrize("name", ["MALAGA_NO_CUDA_GRAPH", "MALAGA_NO_HIP_GRAPH"])
def test_graph_switch_names(tiny, name):
    """The reference's MALAGA_NO_CUDA_GRAPH (src/graph.rs:184) and this backend's
    MALAGA_NO_HIP_GRAPH both turn capture off; "0" keeps it on."""
    path, orc = tiny
    src = pipeline_sentences()[:2]
    for value, capture in (("1", False), ("0", True)):
        gpu = load_with_env(path, **{name: value})
        try:
            assert gpu.generate(src, PLT, opts()) == oracle_rows(orc, src)
            assert gpu.graph_stats()["capture"] is capture
            assert (gpu.graph_stats()["graphs"] > 0) is capture
        finally:
            gpu.close()


def test_chunks_of_max_batch_in_length_order(tiny):
    """Eight sentences with max_batch 3: length-sorted chunks of 3, 3 and 2 sentences
    (src/translator.rs:141-148), hence state buckets b = 4 and b = 2 and no larger one;
    rows come back in input order."""
    path, orc = tiny
    gpu = load_with_env(path)
    src = pipeline_sentences() + [[254, 5, 6, 2], [254] + list(range(10, 24)) + [2]]
    try:
        got = gpu.generate(src, PLT, opts(max_batch=3))
        assert got == oracle_rows(orc, src, max_batch=3)
        assert got == oracle_rows(orc, src)  # chunking does not change any sentence
        assert sorted({k[0] for k in gpu.graph_keys()}) == [2, 4]
    finally:
        gpu.close()


def test_out_of_memory_halves_the_batch(tiny):
    """An allocation failure inside mlg_generate (the first allocation: the encoder's) with
    max_batch 8: translate_batch frees the cached graphs and retries with batches of 4
    (src/translator.rs:150-158), so all states are b = 4 buckets, and the tokens are
    those of an undisturbed run."""
    path, orc = tiny
    gpu = load_with_env(path)
    src = pipeline_sentences() + [[254, 5, 6, 2], [254] + list(range(10, 24)) + [2]]
    want = oracle_rows(orc, src)
    try:
        assert gpu.generate(src, PLT, opts(max_batch=8)) == want
        assert [k[0] for k in gpu.graph_keys()] == [8]
        lib = _lib.load()
        lib.mlg_debug_fail_alloc_after(0)
        try:
            got = gpu.generate(src, PLT, opts(max_batch=8))
        finally:
            lib.mlg_debug_fail_alloc_after(-1)
        assert got == want
        assert {k[0] for k in gpu.graph_keys()} == {4}  # the b = 8 entry was cleared
        assert gpu.graph_stats()["capture"] is True  # only the graph path's own OOM disables capture
    finally:
        gpu.close()


def test_out_of_memory_at_batch_one_is_an_error(tiny):
    """With max_batch 1 there is nothing to halve: the error reaches the caller with the
    "OUT_OF_MEMORY" marker the reference's is_oom matches (src/translator.rs:338-340)."""
    path, _ = tiny
    gpu = load_with_env(path)
    lib = _lib.load()
    try:
        lib.mlg_debug_fail_alloc_after(0)
        with pytest.raises(M.MalagaError) as e:
            gpu.generate(pipeline_sentences()[:2], PLT, opts(max_batch=1))
        assert e.value.code == _lib.ERR_OOM
        assert "OUT_OF_MEMORY" in str(e.value)
    finally:
        lib.mlg_debug_fail_alloc_after(-1)
        gpu.close()


def test_beam_rejects_max_new_past_the_position_table(tiny):
    """Beam search writes K/V slot max_new and reads position max_new + pad + 1, which
    exist up to max_position_embeddings - 2 (the cap of src/translator.rs:181-182): a
    larger max_new is refused before anything runs; the cap itself decodes."""
    path, _ = tiny
    gpu = load_with_env(path)
    try:
        cap = gpu.cfg["max_position_embeddings"] - 2
        src = pipeline_sentences()[:2]
        batch = gpu.encode_cross(src)
        with pytest.raises(M.MalagaError) as e:
            gpu.beam(batch, PLT, max_new=cap + 1, beam_size=2)
        assert e.value.code == _lib.ERR_INVALID
        rows = gpu.beam(batch, PLT, max_new=cap, beam_size=2)
        assert len(rows) == 2 and all(len(r) <= cap for r in rows)
    finally:
        gpu.close()
