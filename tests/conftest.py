"""Shared fixtures.  GPU tests are marked ``gpu``; everything else runs on the CPU."""
from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("models")


def _tiny(model_dir, preset: str) -> Path:
    import malaga_amd as M

    p = model_dir / f"tiny-{preset}.gguf"
    if not p.exists():
        M.write_synthetic(p, M.tiny_config(), preset, M.INIT_TESTUTIL, seed=7, name="tiny")
    return p


@pytest.fixture(scope="session")
def tiny_gguf(model_dir):
    """src/testutil.rs tiny checkpoint (seed 7, pipeline.rs:13) converted per preset."""
    return lambda preset: _tiny(model_dir, preset)


KQ_CONFIG = dict(vocab_size=1000, d_model=256, encoder_layers=2, decoder_layers=2, encoder_heads=4, decoder_heads=4,
                 encoder_ffn=512, decoder_ffn=512, max_position_embeddings=128, max_length=64, scale_embedding=1,
                 bos_token_id=0, pad_token_id=1, eos_token_id=2, decoder_start_token_id=2)


@pytest.fixture(scope="session")
def kq_gguf(model_dir):
    """Parity fixture with d = 256 so that k-quants apply (non-zero biases, gamma, beta)."""
    import malaga_amd as M

    def make(preset: str) -> Path:
        p = model_dir / f"kq-{preset}.gguf"
        if not p.exists():
            M.write_synthetic(p, KQ_CONFIG, preset, M.INIT_NORMAL_RICH, seed=11, std=0.05, name="kq")
        return p

    return make


def golden_sources():
    g = np.load(GOLDEN / "tiny_m2m100.npz")
    src, o = [], 0
    for n in g["src_lens"]:
        src.append(g["src_ids"][o: o + n].tolist())
        o += int(n)
    return g, src


def pipeline_sentences(vocab_words: int = 250, src_lang: int = 254, eos: int = 2):
    """src/testutil.rs:103-106 sentence(n, seed) as word ids, for n = 3 + 4i (pipeline.rs:31-33),
    encoded as [src_lang] toks [eos] (src/translator.rs:90-98)."""
    out = []
    for i in range(6):
        n = 3 + 4 * i
        toks = [4 + (i * 31 + k * 17) % vocab_words for k in range(n)]
        out.append([src_lang] + toks + [eos])
    return out
