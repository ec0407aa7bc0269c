"""End-to-end parity of the HIP decode path with the CPU oracle (tokens bit-exact,
logits within 2e-3 max-abs), mirroring core/tests/pipeline.rs:105-124."""
import numpy as np
import pytest

import malaga_amd as M
import oracle as O
from tests.conftest import golden_sources, pipeline_sentences

pytestmark = pytest.mark.gpu
PLT = 256  # plt_Latn in the tiny vocabulary


@pytest.fixture(scope="module")
def models():
    cache = {}

    def get(path):
        key = str(path)
        if key not in cache:
            cache[key] = (M.Translator.load(path), O.Model(path))
        return cache[key]

    return get


@pytest.mark.parametrize("preset", ["f32", "f16", "q8_0", "q4_k_m"])
def test_fused_greedy_matches_oracle_tiny(tiny_gguf, models, preset):
    gpu, orc = models(tiny_gguf(preset))
    src = pipeline_sentences()
    want, gap = orc.translate_batch(src, PLT, kv_f16=True)
    got = gpu.generate(src, PLT)
    assert got == want, f"min top-2 gap {gap}"
    # the second run replays the cached graphs (pipeline.rs:121-122)
    assert gpu.generate(src, PLT) == got
    assert gpu.graph_stats()["graphs"] >= 1
    # fused = false: the generic decoder (f32 K/V, src/translator.rs:195-199), against the
    # oracle's f32-K/V decode; on this fixture it also equals the fused decode
    # (pipeline.rs:105-124)
    want32, _ = orc.translate_batch(src, PLT, kv_f16=False)
    assert gpu.generate(src, PLT, M.GenOptions(fused=False)) == want32 == got


@pytest.mark.parametrize("preset", ["f32", "q8_0"])
def test_fused_f16_kv_matches_f32_generic_path(tiny_gguf, models, preset):
    """pipeline.rs:105-124: fused GPU (f16 KV) == generic path (f32 KV), F32 and Q8_0."""
    gpu, orc = models(tiny_gguf(preset))
    src = pipeline_sentences()
    want, _ = orc.translate_batch(src, PLT, kv_f16=False)
    assert gpu.generate(src, PLT) == want


@pytest.mark.parametrize("preset", ["q4_k_m", "q5_k_m", "q6_k", "q8_0", "f16"])
def test_kquant_fixture_tokens_and_logits(kq_gguf, models, preset):
    gpu, orc = models(kq_gguf(preset))
    rng = np.random.default_rng(5)
    src = [[997] + rng.integers(4, 990, n).tolist() + [2] for n in (30, 11, 3, 20)]
    want, gap = orc.translate_batch(src, 998, kv_f16=True)
    got = gpu.generate(src, 998)
    assert got == want, f"min top-2 gap {gap}"
    T = 10
    tgt = np.zeros((len(src), T), np.uint32)
    tgt[:, 0], tgt[:, 1] = 2, 998
    tgt[:, 2:] = rng.integers(4, 990, (len(src), T - 2))
    lg_gpu = gpu.teacher_forced_logits(src, tgt)
    lg_orc = orc.teacher_forced_logits(src, tgt, kv_f16=True)
    assert np.abs(lg_gpu - lg_orc).max() < 2e-3


def test_logits_match_transformers_golden(tiny_gguf, models):
    """GPU logits against the Hugging Face golden vectors (f32 KV there, f16 here)."""
    g, src = golden_sources()
    gpu, _ = models(tiny_gguf("f32"))
    lg = gpu.teacher_forced_logits(src, g["tgt"])
    assert np.abs(lg - g["logits_f32"]).max() < 2e-2
    assert (lg.argmax(-1) == g["logits_f32"].argmax(-1)).mean() > 0.97


@pytest.mark.parametrize("k", [1, 2, 4])
def test_beam_matches_oracle(tiny_gguf, kq_gguf, models, k):
    for path, tgt in ((tiny_gguf("f32"), PLT), (kq_gguf("q4_k_m"), 998)):
        gpu, orc = models(path)
        src = pipeline_sentences()[:4] if tgt == PLT else [[997, 5, 6, 7, 8, 2], [997, 40, 2]]
        # beam search decodes on f32 K/V, as the reference's Nllb::decode (src/model.rs:195-227)
        want, _ = orc.translate_batch(src, tgt, beam_size=k, kv_f16=False)
        got = gpu.generate(src, tgt, M.GenOptions(beam_size=k))
        assert got == want
    if k == 1:
        assert got == gpu.generate(src, tgt)  # beam 1 == greedy (pipeline.rs:59-69)


@pytest.mark.parametrize("preset", ["f32", "q8_0"])
def test_wide_beam_is_exhaustive_search(model_dir, models, preset):
    """Beam 8 over a vocabulary of 8 for two steps prunes nothing, so the GPU's beam
    search must return the best of all hypotheses (tests/test_oracle_beam.py), at
    length penalties under which hypotheses of 0, 1 and 2 tokens win."""
    from tests.test_oracle_beam import PENALTIES, WIDE_SOURCES, WIDE_TGT, exhaustive, wide_model

    gpu, orc = models(wide_model(model_dir, preset))
    for p in PENALTIES:
        opts = M.GenOptions(beam_size=8, max_new_tokens=2, length_penalty=p)
        for graph in (True, False):
            opts.fused = graph
            got = gpu.generate(WIDE_SOURCES, WIDE_TGT, opts)
            for src, row in zip(WIDE_SOURCES, got):
                want, gap = exhaustive(orc, src, WIDE_TGT, p, kv_f16=False)  # beam runs on f32 K/V
                assert gap > 1e-3
                assert row == want, (src, p, graph)


def test_beam_graph_replay_matches_eager(kq_gguf, models):
    """The beam step is one captured step + top-k replayed every step; eager calls
    between the graph calls check that every replay gives the eager tokens."""
    gpu, _ = models(kq_gguf("q4_k_m"))
    src = [[997, 5, 6, 7, 8, 2], [997, 40, 2], [997] + list(range(10, 30)) + [2]]
    graph = M.GenOptions(beam_size=4, max_new_tokens=14)
    eager = M.GenOptions(beam_size=4, max_new_tokens=14, fused=False)
    want = gpu.generate(src, 998, eager)
    for _ in range(3):
        assert gpu.generate(src, 998, graph) == want
        assert gpu.generate(src[:2], 998, eager) == want[:2]


def test_batching_does_not_change_translations_gpu(tiny_gguf, models):
    gpu, _ = models(tiny_gguf("f32"))
    src = pipeline_sentences()
    batched = gpu.generate(src, PLT)
    for s, b in zip(src, batched):
        assert gpu.generate([s], PLT) == [b]


def test_eos_mask_and_budget(kq_gguf, models):
    gpu, orc = models(kq_gguf("q4_k_m"))
    src = [[997, 5, 6, 2], [997] + list(range(10, 40)) + [2]]
    got = gpu.generate(src, 998, M.GenOptions(eos_mask=True, max_new_tokens=12))
    want, _ = orc.generate(src, 998, max_new_tokens=12, eos_mask=True)
    assert got == want and all(len(r) == 12 for r in got)


def test_oom_falls_back_to_eager_and_keeps_tokens(tiny_gguf, models):
    """src/graph.rs:214-222 forced from the host: an injected allocation failure inside
    the graph path disables capture; the retry decodes eagerly with the same tokens."""
    from malaga_amd import _lib

    gpu, orc = models(tiny_gguf("q8_0"))
    src = pipeline_sentences()[:3]
    want, _ = orc.translate_batch(src, PLT, kv_f16=True)
    gpu.clear_graphs()
    batch = gpu.encode_cross(src)
    _lib.load().mlg_debug_fail_alloc_after(0)
    try:
        got = gpu.greedy(batch, PLT, max_new=gpu.budget(max(len(s) for s in src)))
    finally:
        _lib.load().mlg_debug_fail_alloc_after(-1)
    assert [r[: gpu.budget(len(s))] for r, s in zip(got, src)] == want
    assert gpu.graph_stats()["capture"] is False


@pytest.fixture(scope="module")
def unfused_models():
    """Second Translator per file with the unfused step (MALAGA_NO_FUSED_STEP=1)."""
    import os

    cache = {}

    def get(path):
        key = str(path)
        if key not in cache:
            os.environ["MALAGA_NO_FUSED_STEP"] = "1"
            try:
                cache[key] = M.Translator.load(path)
            finally:
                del os.environ["MALAGA_NO_FUSED_STEP"]
        return cache[key]

    return get


@pytest.mark.parametrize("preset", ["f32", "f16", "q8_0"])
@pytest.mark.parametrize("nb", [1, 2, 4])
def test_fused_step_small_batches_tiny(tiny_gguf, models, unfused_models, preset, nb):
    """Batches of <= 4 rows run the fused step kernels (k_step.hip)."""
    gpu, orc = models(tiny_gguf(preset))
    src = pipeline_sentences()[:nb]
    want, gap = orc.translate_batch(src, PLT, kv_f16=True)
    assert gpu.generate(src, PLT) == want, f"min gap {gap}"
    want32, _ = orc.translate_batch(src, PLT, kv_f16=False)
    assert gpu.generate(src, PLT, M.GenOptions(fused=False)) == want32  # the generic decoder
    assert unfused_models(tiny_gguf(preset)).generate(src, PLT) == want
    T = 9
    rng = np.random.default_rng(nb)
    tgt = np.zeros((nb, T), np.uint32)
    tgt[:, 0], tgt[:, 1] = 2, PLT
    tgt[:, 2:] = rng.integers(4, 254, (nb, T - 2))
    lg = gpu.teacher_forced_logits(src, tgt)
    assert np.abs(lg - orc.teacher_forced_logits(src, tgt, kv_f16=True)).max() < 2e-3
    # The two paths sum in different orders; an f32 difference of one rounding can
    # move a K/V value across an f16 rounding boundary (5e-4 relative), so the
    # paths agree to ~1e-4 rather than to f32 rounding.
    assert np.abs(lg - unfused_models(tiny_gguf(preset)).teacher_forced_logits(src, tgt)).max() < 1e-3


@pytest.mark.parametrize("preset", ["q4_k_m", "q5_k_m", "q6_k", "q8_0"])
@pytest.mark.parametrize("nb", [1, 2])
def test_fused_step_small_batches_kquant(kq_gguf, models, unfused_models, preset, nb):
    gpu, orc = models(kq_gguf(preset))
    rng = np.random.default_rng(100 + nb)
    src = [[997] + rng.integers(4, 990, n).tolist() + [2] for n in (25, 7)[:nb]]
    want, gap = orc.translate_batch(src, 998, kv_f16=True)
    assert gpu.generate(src, 998) == want, f"min gap {gap}"
    assert unfused_models(kq_gguf(preset)).generate(src, 998) == want
    T = 12
    tgt = np.zeros((nb, T), np.uint32)
    tgt[:, 0], tgt[:, 1] = 2, 998
    tgt[:, 2:] = rng.integers(4, 990, (nb, T - 2))
    lg = gpu.teacher_forced_logits(src, tgt)
    assert np.abs(lg - orc.teacher_forced_logits(src, tgt, kv_f16=True)).max() < 2e-3


@pytest.mark.parametrize("preset", ["q4_k_m", "q5_k_m"])
@pytest.mark.parametrize("nb", [1, 2])
def test_fused_cross_attention_equals_split_kernels(kq_gguf, models, preset, nb):
    """k_xattn (cross_q + cross attention + out-projection slice in one launch) against
    the same step with the two launches (MALAGA_SPLIT_CROSS_STEP=1): every sum is in the
    same order, so the logits are equal bit for bit."""
    import os

    gpu, _ = models(kq_gguf(preset))
    os.environ["MALAGA_SPLIT_CROSS_STEP"] = "1"
    try:
        split = M.Translator.load(kq_gguf(preset))
    finally:
        del os.environ["MALAGA_SPLIT_CROSS_STEP"]
    rng = np.random.default_rng(300 + nb)
    src = [[997] + rng.integers(4, 990, n).tolist() + [2] for n in (19, 40)[:nb]]
    T = 10
    tgt = np.zeros((nb, T), np.uint32)
    tgt[:, 0], tgt[:, 1] = 2, 998
    tgt[:, 2:] = rng.integers(4, 990, (nb, T - 2))
    try:
        assert np.array_equal(gpu.teacher_forced_logits(src, tgt), split.teacher_forced_logits(src, tgt))
        assert gpu.generate(src, 998) == split.generate(src, 998)
    finally:
        split.close()


@pytest.mark.parametrize("preset", ["q4_k_m", "q6_k", "q8_0"])
@pytest.mark.parametrize("nb", [7, 33])
def test_batched_fused_cross_attention(kq_gguf, models, preset, nb):
    """k_dxattn (batches of 5..64 rows, heads of 64: cross_q with the cross LayerNorm and
    the cross attention in one launch, 2 rows x 1 head per workgroup, 4 waves per (row,
    head) pair) against the same steps with the two launches (MALAGA_SPLIT_CROSS_STEP=1):
    q adds the same partials in the same order as k_dgemm and the attention takes the same
    keys in the same order as k_attn_waves, so the logits are equal bit for bit.  7 rows
    leave a partial row pair; 33 pad to 64 rows; beam 4 over two sentences gives 8 rows."""
    import os

    gpu, orc = models(kq_gguf(preset))
    os.environ["MALAGA_SPLIT_CROSS_STEP"] = "1"
    try:
        split = M.Translator.load(kq_gguf(preset))
    finally:
        del os.environ["MALAGA_SPLIT_CROSS_STEP"]
    rng = np.random.default_rng(400 + nb)
    src = [[997] + rng.integers(4, 990, int(n)).tolist() + [2] for n in rng.integers(2, 60, nb)]
    T = 8
    tgt = np.zeros((nb, T), np.uint32)
    tgt[:, 0], tgt[:, 1] = 2, 998
    tgt[:, 2:] = rng.integers(4, 990, (nb, T - 2))
    try:
        lg = gpu.teacher_forced_logits(src, tgt)
        assert np.array_equal(lg, split.teacher_forced_logits(src, tgt))
        assert np.abs(lg - orc.teacher_forced_logits(src, tgt, kv_f16=True)).max() < 2e-3
        # the generic decoder's f32 K/V through the same two forms (beam search runs it)
        lg32 = gpu.teacher_forced_logits(src, tgt, kv_f32=True)
        assert np.array_equal(lg32, split.teacher_forced_logits(src, tgt, kv_f32=True))
        assert np.abs(lg32 - orc.teacher_forced_logits(src, tgt, kv_f16=False)).max() < 2e-3
        want, gap = orc.translate_batch(src, 998, max_batch=64, kv_f16=True, max_new_tokens=10)
        got = gpu.generate(src, 998, M.GenOptions(max_new_tokens=10, max_batch=64))
        assert got == want, f"min top-2 gap {gap}"
        assert split.generate(src, 998, M.GenOptions(max_new_tokens=10, max_batch=64)) == want
        opts = M.GenOptions(beam_size=4, max_new_tokens=8, max_batch=8)
        assert gpu.generate(src[:2], 998, opts) == split.generate(src[:2], 998, opts)
    finally:
        split.close()


@pytest.mark.parametrize("preset", ["q4_k_m", "q5_k_m", "q6_k", "q8_0", "f16"])
@pytest.mark.parametrize("nb", [7, 16, 33])
def test_batched_decode_mfma_path(kq_gguf, models, preset, nb):
    """Batches above the register GEMV (> 4 rows): MFMA GEMMs with split-K reductions
    fused with the residual + LayerNorm and the QKV split, the batched LM head
    (argmax partials on the MFMA units up to 32 rows, logits + argmax above)."""
    gpu, orc = models(kq_gguf(preset))
    rng = np.random.default_rng(200 + nb)
    src = [[997] + rng.integers(4, 990, int(n)).tolist() + [2] for n in rng.integers(2, 40, nb)]
    want, gap = orc.translate_batch(src, 998, max_batch=64, kv_f16=True, max_new_tokens=10)
    got = gpu.generate(src, 998, M.GenOptions(max_new_tokens=10, max_batch=64))
    assert got == want, f"min top-2 gap {gap}"
    T = 8
    tgt = np.zeros((nb, T), np.uint32)
    tgt[:, 0], tgt[:, 1] = 2, 998
    tgt[:, 2:] = rng.integers(4, 990, (nb, T - 2))
    lg = gpu.teacher_forced_logits(src, tgt)
    assert np.abs(lg - orc.teacher_forced_logits(src, tgt, kv_f16=True)).max() < 2e-3


@pytest.mark.parametrize("preset", ["q4_k_m", "q6_k"])
def test_cross_kv_in_layer_chunks(kq_gguf, models, preset, monkeypatch):
    """The encoder computes the stacked cross K/V of several decoder layers per GEMM while
    its f32 staging fits a budget; past it, later chunks read row views of the stacked
    matrix (their planes and tile-major copies from the chunk's first row on).  With the
    budget at 0 every layer is a chunk of its own: same tokens and logits as the oracle."""
    gpu, orc = models(kq_gguf(preset))
    rng = np.random.default_rng(450)
    src = [[997] + rng.integers(4, 990, int(n)).tolist() + [2] for n in rng.integers(2, 40, 16)]
    want, gap = orc.translate_batch(src, 998, max_batch=64, kv_f16=True, max_new_tokens=10)
    T = 8
    tgt = np.zeros((len(src), T), np.uint32)
    tgt[:, 0], tgt[:, 1] = 2, 998
    tgt[:, 2:] = rng.integers(4, 990, (len(src), T - 2))
    monkeypatch.setenv("MALAGA_CROSS_KV_STAGING_MB", "0")
    got = gpu.generate(src, 998, M.GenOptions(max_new_tokens=10, max_batch=64))
    one = gpu.generate(src[:1], 998, M.GenOptions(max_new_tokens=10))
    lg = gpu.teacher_forced_logits(src, tgt)
    monkeypatch.delenv("MALAGA_CROSS_KV_STAGING_MB")
    assert got == want, f"min top-2 gap {gap}"
    assert one == want[:1]
    assert np.abs(lg - orc.teacher_forced_logits(src, tgt, kv_f16=True)).max() < 2e-3


def test_config5_shapes_batch64(model_dir, models):
    """BASELINE config 5 shapes (NLLB-3.3B: d_model 2048, 16 heads of 128, FFN 8192,
    q4_k_m) at two layers and a 4096-token vocabulary so that the oracle finishes in
    seconds; a dynamic batch of 40 sentences (state bucket 64), lognormal lengths."""
    cfg = M.nllb_3b_config()
    cfg.update(vocab_size=4096, encoder_layers=2, decoder_layers=2, max_position_embeddings=256, max_length=64)
    path = model_dir / "c5-q4_k_m.gguf"
    if not path.exists():
        M.write_synthetic(path, cfg, "q4_k_m", M.INIT_NORMAL_RICH, seed=5, std=0.02, name="config5-shape")
    gpu, orc = models(path)
    rng = np.random.default_rng(55)
    lens = np.clip(np.rint(rng.lognormal(np.log(12) - 0.125, 0.5, 40)), 3, 40).astype(int)
    src = [[4000] + rng.integers(4, 3990, int(n)).tolist() + [2] for n in lens]
    want, gap = orc.translate_batch(src, 4001, max_batch=64, kv_f16=True, max_new_tokens=6)
    got = gpu.generate(src, 4001, M.GenOptions(max_new_tokens=6, max_batch=64))
    assert got == want, f"min top-2 gap {gap}"
    # batch of 3: the fused step at d = 2048 (hd = 128, head groups of 2)
    want3, gap3 = orc.translate_batch(src[:3], 4001, kv_f16=True, max_new_tokens=6)
    assert gpu.generate(src[:3], 4001, M.GenOptions(max_new_tokens=6)) == want3, f"min top-2 gap {gap3}"


@pytest.mark.parametrize("preset", ["q4_k_m", "q6_k", "q8_0"])
def test_decode_gemm_step_equals_split_k_step(kq_gguf, models, preset):
    """Batches of 5..64 rows run the decode GEMMs (k_dgemm.hip: LayerNorm statistics
    carried with the residual stream, no split K); MALAGA_SPLIT_K_STEP=1 keeps the
    split-K GEMMs with their reduction kernels.  Same tokens; logits within the f32
    reordering of the sums (plus f16 K/V rounding flips, as for the fused step)."""
    import os

    gpu, orc = models(kq_gguf(preset))
    os.environ["MALAGA_SPLIT_K_STEP"] = "1"
    try:
        split = M.Translator.load(kq_gguf(preset))
    finally:
        del os.environ["MALAGA_SPLIT_K_STEP"]
    rng = np.random.default_rng(400)
    try:
        for nb in (5, 33, 64):
            src = [[997] + rng.integers(4, 990, int(n)).tolist() + [2] for n in rng.integers(2, 40, nb)]
            opts = M.GenOptions(max_new_tokens=8, max_batch=64)
            assert gpu.generate(src, 998, opts) == split.generate(src, 998, opts)
            T = 6
            tgt = np.zeros((nb, T), np.uint32)
            tgt[:, 0], tgt[:, 1] = 2, 998
            tgt[:, 2:] = rng.integers(4, 990, (nb, T - 2))
            a, b = gpu.teacher_forced_logits(src, tgt), split.teacher_forced_logits(src, tgt)
            assert np.abs(a - b).max() < 1e-3
            assert np.abs(a - orc.teacher_forced_logits(src, tgt, kv_f16=True)).max() < 2e-3
    finally:
        split.close()


def test_activation_beyond_f16_range_is_an_error(model_dir):
    """The MFMA products take their activations as f16 hi + lo, which holds |x| < 65520.
    A checkpoint whose activations go past that (N(0, 2000) weights: attention outputs and
    FFN activations ~1e5) must end in an error that says so, for greedy and beam alike,
    never in tokens decoded from NaN logits.  (The reference keeps f32 activations; this is
    the documented range of this backend.)"""
    from tests.conftest import KQ_CONFIG

    p = model_dir / "huge-q8_0.gguf"
    if not p.exists():
        M.write_synthetic(p, KQ_CONFIG, "q8_0", M.INIT_NORMAL, seed=3, std=2000.0, name="huge")
    gpu = M.Translator.load(p)
    try:
        src = [[997, 5 + i, 6, 2] for i in range(8)]
        for opts in (M.GenOptions(max_new_tokens=4, max_batch=8),
                     M.GenOptions(max_new_tokens=4, max_batch=8, beam_size=2)):
            with pytest.raises(M.MalagaError, match="finite logit"):
                gpu.generate(src, 998, opts)
    finally:
        gpu.close()
