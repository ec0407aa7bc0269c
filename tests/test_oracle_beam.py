"""Pins the oracle's beam search (src/translator.rs:250-358) against exhaustive search.

With beam width k equal to the vocabulary size and max_new = 2, no hypothesis is ever
pruned: step 1 keeps every non-EOS token alive (EOS goes to `done`), and step 2 sends
all k x k continuations to `done` (step == max_new).  The beam result must then be the
best of all one- and two-step hypotheses under the reference's score,
sum of log-probs / len^p with len = tokens + 1 and EOS not counted as a token
(translator.rs:262, 284-292).  The log-probs come from the oracle's teacher-forced
decoder, which is pinned separately against transformers' M2M100 (golden vectors).

The fixture has a vocabulary of 8 and peaky distributions (std 0.5), so that
hypotheses of length 0, 1 and 2 compete at the chosen length penalties and a wrong
length in the penalty, a dropped EOS hypothesis or a wrong pruning rule changes the
answer.  GPU beam search is compared with the same exhaustive answer in
tests/test_gpu_parity.py.
"""
from __future__ import annotations

import numpy as np
import pytest

WIDE_CONFIG = dict(vocab_size=8, d_model=64, encoder_layers=2, decoder_layers=2, encoder_heads=4, decoder_heads=4,
                   encoder_ffn=128, decoder_ffn=128, max_position_embeddings=64, max_length=32, scale_embedding=1,
                   bos_token_id=0, pad_token_id=1, eos_token_id=2, decoder_start_token_id=2)
WIDE_TGT = 7
WIDE_SOURCES = [[7, 2], [6, 5, 2], [4, 4, 3, 2], [3, 3, 3, 7, 2], [6, 7, 5, 6, 7, 2], [6, 6, 5, 5, 7, 4, 2],
                [7, 6, 3, 4, 7, 5, 3, 2], [6, 6, 7, 3, 3, 7, 3, 5, 3, 2]]
PENALTIES = (0.0, 0.5, 1.0, 2.0)


def wide_model(model_dir, preset: str = "f32"):
    import malaga_amd as M

    p = model_dir / f"wide-{preset}.gguf"
    if not p.exists():
        M.write_synthetic(p, WIDE_CONFIG, preset, M.INIT_NORMAL_RICH, seed=20, std=0.5, name="wide")
    return p


def _log_softmax(x: np.ndarray) -> np.ndarray:
    """candle_nn log_softmax (src/model.rs:615-617): (x - max) - ln(sum exp(x - max))."""
    x = x.astype(np.float32)
    m = x.max()
    s = np.exp((x - m).astype(np.float64)).sum()
    return ((x - m) - np.float32(np.log(s))).astype(np.float32)


def exhaustive(orc, src: list[int], tgt: int, p: float, kv_f16: bool = True):
    """All hypotheses of at most two steps, scored as translator.rs:284-292, on the
    oracle's logits with f16 (or, kv_f16=False, f32) K/V.
    Returns (best tokens, score gap between the best and the runner-up)."""
    V, eos, start = WIDE_CONFIG["vocab_size"], WIDE_CONFIG["eos_token_id"], WIDE_CONFIG["decoder_start_token_id"]
    tf = orc.teacher_forced_logits([src] * V, np.array([[start, tgt, t1] for t1 in range(V)], dtype=np.uint32),
                                   kv_f16=kv_f16)
    pen = lambda n: np.float32(max(n, 1)) ** np.float32(p)  # noqa: E731
    lp1 = _log_softmax(tf[0, 1])
    hyps = [(float(np.float32(lp1[eos]) / pen(1)), [])]
    for t1 in range(V):
        if t1 == eos:
            continue
        lp2 = _log_softmax(tf[t1, 2])
        for t2 in range(V):
            toks = [t1] if t2 == eos else [t1, t2]
            s = np.float32(lp1[t1]) + np.float32(lp2[t2])
            hyps.append((float(s / pen(len(toks) + 1)), toks))
    hyps.sort(key=lambda h: -h[0])
    return hyps[0][1], hyps[0][0] - hyps[1][0]


@pytest.fixture(scope="module")
def wide(model_dir):
    import oracle as O

    return O.Model(wide_model(model_dir))


@pytest.mark.parametrize("p", PENALTIES)
def test_wide_beam_is_exhaustive_search(wide, p):
    got, _ = wide.generate(WIDE_SOURCES, WIDE_TGT, beam_size=WIDE_CONFIG["vocab_size"], max_new_tokens=2,
                           length_penalty=p)
    for src, row in zip(WIDE_SOURCES, got):
        want, gap = exhaustive(wide, src, WIDE_TGT, p)
        assert gap > 1e-3, "near tie: the fixture no longer separates the hypotheses"
        assert row == want, (src, p)


def test_wide_fixture_makes_lengths_compete(wide):
    """Across the penalties the exhaustive answers have every length 0, 1 and 2, so the
    comparison above exercises the penalty's length term and the EOS hypotheses."""
    lens = {len(exhaustive(wide, src, WIDE_TGT, p)[0]) for src in WIDE_SOURCES for p in PENALTIES}
    assert lens == {0, 1, 2}, lens


def test_narrow_beam_prunes(wide):
    """Control: beam 1 over the same fixture prunes, and differs from exhaustive search
    somewhere (otherwise the wide comparison would be vacuous)."""
    diff = 0
    for p in PENALTIES:
        got, _ = wide.generate(WIDE_SOURCES, WIDE_TGT, beam_size=1, max_new_tokens=2, length_penalty=p)
        diff += sum(row != exhaustive(wide, src, WIDE_TGT, p)[0] for src, row in zip(WIDE_SOURCES, got))
    assert diff > 0
