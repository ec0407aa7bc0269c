"""The CPU oracle against known answers it does not compute itself.

* Hugging Face transformers' M2M100 logits on the tiny test checkpoint
  (tests/golden/make_golden.py): pins the forward pass, the converter's layout
  (fused QKV, 1/sqrt(hd) pre-scale, tied embedding) and the Q8_0 codec.
* transformers' greedy search on the same checkpoint: pins the greedy decode loop.
* src/testutil.rs:57-69 xorshift stream (Python integer restatement).
* src/model.rs:324-340 sinusoidal table against its closed form.
"""
import numpy as np
import pytest

import oracle as O
from tests.conftest import golden_sources


@pytest.mark.parametrize("preset,key", [("f32", "logits_f32"), ("q8_0", "logits_q8_0")])
def test_logits_match_transformers_m2m100(tiny_gguf, preset, key):
    g, src = golden_sources()
    m = O.Model(tiny_gguf(preset))
    lg = m.teacher_forced_logits(src, g["tgt"], kv_f16=False)
    ref = g[key]
    # f32 reference vs f64-accumulated oracle; logits up to ~14 in magnitude
    assert np.abs(lg - ref).max() < 5e-5
    # the argmax at every position agrees (what greedy decoding consumes)
    assert (lg.argmax(-1) == ref.argmax(-1)).all()


@pytest.mark.parametrize("tgt_lang", [255, 256])
def test_greedy_matches_transformers_generate(tiny_gguf, tgt_lang):
    """Greedy decoding with the target language forced after decoder_start
    (src/translator.rs:214-241, src/graph.rs:255-297) against transformers' greedy
    search on the same checkpoint (EOS masking off, 20 tokens, f32 caches)."""
    g, src = golden_sources()
    want = g[f"greedy_{tgt_lang}_20"]
    m = O.Model(tiny_gguf("f32"))
    for i, s in enumerate(src):
        rows, _ = m.generate([s], tgt_lang, max_new_tokens=20, kv_f16=False)
        ref = [int(t) for t in want[i] if t >= 0]
        assert rows[0] == ref, (i, rows[0], ref)


def test_encoder_output_matches_transformers(tiny_gguf):
    g, src = golden_sources()
    m = O.Model(tiny_gguf("f32"))
    enc = m.encoder_output(src)
    for i, n in enumerate(g["src_lens"]):
        assert np.abs(enc[i, :n] - g["encoder_out"][i, :n]).max() < 1e-5


def test_f16_kv_rounding_changes_little(tiny_gguf):
    """The fused path stores K/V in f16 (kernels/malaga.cu:151-152): the oracle's
    emulation must stay close to the f32 cache and actually round."""
    g, src = golden_sources()
    m = O.Model(tiny_gguf("f32"))
    a = m.teacher_forced_logits(src, g["tgt"], kv_f16=False)
    b = m.teacher_forced_logits(src, g["tgt"], kv_f16=True)
    d = np.abs(a - b).max()
    assert 0 < d < 2e-2


def test_xorshift_stream_matches_the_python_restatement(tiny_gguf):
    """First embedding values of the C++ testutil generator (F32 preset keeps them exact)."""
    from malaga_amd.gguf import read_gguf

    g, _ = golden_sources()
    _, meta, tensors, data = read_gguf(tiny_gguf("f32"))
    t = tensors["token_embd.weight"]
    first = np.frombuffer(data, dtype=np.float32, count=8, offset=t["data_start"])
    np.testing.assert_array_equal(first, g["xorshift_seed7_scale05"])


def test_sinusoidal_table_closed_form():
    n, d, pad = 40, 64, 1
    tab = O.sinusoidal_table(n, d, pad)
    half = d // 2
    p = np.arange(n)[:, None].astype(np.float64)
    f = np.exp(-np.arange(half) * np.log(10000.0) / (half - 1))[None, :]
    ref = np.concatenate([np.sin(p * f), np.cos(p * f)], axis=1).astype(np.float32)
    ref[pad] = 0
    np.testing.assert_allclose(tab, ref, atol=1e-6)
    assert (tab[pad] == 0).all() and tab[0, half] == 1.0  # cos(0)
