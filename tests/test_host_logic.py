"""Host-side logic with reference known answers and the oracle's decoding invariants."""
import numpy as np

import malaga_amd as M
import oracle as O
from tests.conftest import pipeline_sentences


def test_bucket_known_answers():
    """src/graph.rs:372-379."""
    assert M.bucket(5, 16, 1024) == 16
    assert M.bucket(17, 16, 1024) == 32
    assert M.bucket(64, 32, 1024) == 64
    assert M.bucket(900, 32, 512) == 900


def test_budget_rule(tiny_gguf):
    """src/translator.rs:181-182: 2*len + 16 clamped to [1, min(max_length, max_pos - 2)]."""
    m = O.Model(tiny_gguf("f32"))
    assert m.budget(5) == 26
    assert m.budget(40) == 64  # max_length 64
    assert m.budget(5, 3) == 3


def test_batching_does_not_change_translations(tiny_gguf):
    """pipeline.rs:44-57 (REQ-INF-002) on the oracle, f32."""
    m = O.Model(tiny_gguf("f32"))
    src = pipeline_sentences()
    batched, _ = m.translate_batch(src, 256, kv_f16=False)
    for s, b in zip(src, batched):
        single, _ = m.generate([s], 256, kv_f16=False)
        assert single[0] == b


def test_beam1_is_greedy_and_beam_is_deterministic(tiny_gguf):
    """pipeline.rs:59-69 (REQ-INF-003) on the oracle."""
    m = O.Model(tiny_gguf("f32"))
    s = [pipeline_sentences()[2]]
    greedy, _ = m.generate(s, 256, kv_f16=False)
    b1, _ = m.generate(s, 256, beam_size=1, kv_f16=False)
    assert b1 == greedy
    b3a, _ = m.generate(s, 256, beam_size=3, kv_f16=False)
    b3b, _ = m.generate(s, 256, beam_size=3, kv_f16=False)
    assert b3a == b3b


def test_eos_mask_fixes_lengths(tiny_gguf):
    m = O.Model(tiny_gguf("f32"))
    src = pipeline_sentences()[:3]
    rows, _ = m.generate(src, 256, eos_mask=True)
    for s, r in zip(src, rows):
        assert len(r) == m.budget(len(s)) and 2 not in r
