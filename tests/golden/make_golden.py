"""Writes tests/golden/tiny_m2m100.npz: known-answer vectors for the oracle.

Run in the build container only (needs transformers, not the reference):
    python tests/golden/make_golden.py

What it pins, independently of oracle/oracle.c:
  * src/testutil.rs:56-69 xorshift weights: first values of the stream, restated
    here in Python integer arithmetic.
  * The whole forward pass (embedding scale, sinusoidal positions, pre-LN
    encoder/decoder layers, 1/sqrt(hd) scaling, ReLU FFN, final norms, tied LM
    head): logits of Hugging Face transformers' M2M100ForConditionalGeneration
    (the model the reference validated against, spec/manual-tests.md MT-01) on
    the tiny test checkpoint, for teacher-forced target sequences.
  * Greedy decoding (src/translator.rs:214-241): transformers' greedy search with
    the target language forced as the first generated token, 20 tokens per source,
    for target languages 255 and 256.
  * Q8_0: the same logits with every projection weight replaced by its Q8_0
    round trip (closed form: d = f16(amax / 127), q = round-half-away(x / d)),
    which pins the converter's Q8_0 quantizer and the oracle's Q8_0 dequantizer.
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "tiny_m2m100.npz"

# src/testutil.rs:18-30
V, D, H, FFN, LAYERS, MAXPOS, WORDS = 257, 64, 4, 128, 2, 128, 250


def xorshift_stream(seed: int):
    """src/testutil.rs:57-69 in Python integers."""
    mask = (1 << 64) - 1
    state = ((seed * 0x9E3779B97F4A7C15) & mask) | 1

    def draw(n: int, scale: float) -> np.ndarray:
        nonlocal state
        out = np.empty(n, dtype=np.float32)
        for i in range(n):
            state ^= (state << 13) & mask
            state ^= state >> 7
            state ^= (state << 17) & mask
            v = np.float32(state >> 40) / np.float32(1 << 24)
            out[i] = (v - np.float32(0.5)) * np.float32(2.0) * np.float32(scale)
        return out

    return draw


def tiny_weights(seed: int = 7) -> dict:
    """HF-named tensors in the draw order of src/testutil.rs:70-98."""
    draw = xorshift_stream(seed)
    w = {"model.shared.weight": draw(V * D, 0.5).reshape(V, D)}
    ones, zeros = np.ones(D, np.float32), np.zeros(D, np.float32)
    for side in ("encoder", "decoder"):
        for l in range(LAYERS):
            p = f"model.{side}.layers.{l}"
            attns = ["self_attn"] + (["encoder_attn"] if side == "decoder" else [])
            for a in attns:
                for proj in ("q_proj", "k_proj", "v_proj", "out_proj"):
                    w[f"{p}.{a}.{proj}.weight"] = draw(D * D, 0.3).reshape(D, D)
                    w[f"{p}.{a}.{proj}.bias"] = draw(D, 0.1)
                w[f"{p}.{a}_layer_norm.weight"] = ones.copy()
                w[f"{p}.{a}_layer_norm.bias"] = zeros.copy()
            w[f"{p}.fc1.weight"] = draw(FFN * D, 0.3).reshape(FFN, D)
            w[f"{p}.fc1.bias"] = draw(FFN, 0.1)
            w[f"{p}.fc2.weight"] = draw(D * FFN, 0.3).reshape(D, FFN)
            w[f"{p}.fc2.bias"] = draw(D, 0.1)
            w[f"{p}.final_layer_norm.weight"] = ones.copy()
            w[f"{p}.final_layer_norm.bias"] = zeros.copy()
        w[f"model.{side}.layer_norm.weight"] = ones.copy()
        w[f"model.{side}.layer_norm.bias"] = zeros.copy()
    return w


def q8_0_roundtrip(x: np.ndarray) -> np.ndarray:
    """Q8_0 closed form on rows of 32: d = f16(amax/127); q = round half away from zero."""
    flat = x.astype(np.float32).reshape(-1, 32)
    amax = np.abs(flat).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    v = flat * inv[:, None]
    q = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)
    d16 = d.astype(np.float16).astype(np.float32)
    return (d16[:, None] * q.astype(np.float32)).reshape(x.shape)


def hf_logits(weights: dict, src: list[list[int]], tgt: np.ndarray):
    from transformers import M2M100Config, M2M100ForConditionalGeneration

    cfg = M2M100Config(vocab_size=V, d_model=D, encoder_layers=LAYERS, decoder_layers=LAYERS,
                       encoder_attention_heads=H, decoder_attention_heads=H, encoder_ffn_dim=FFN,
                       decoder_ffn_dim=FFN, max_position_embeddings=MAXPOS, scale_embedding=True,
                       activation_function="relu", dropout=0.0, attention_dropout=0.0, activation_dropout=0.0,
                       encoder_layerdrop=0.0, decoder_layerdrop=0.0, pad_token_id=1, bos_token_id=0,
                       eos_token_id=2, decoder_start_token_id=2, tie_word_embeddings=True)
    cfg._attn_implementation = "eager"
    model = M2M100ForConditionalGeneration(cfg).eval()
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in weights.items()}
    sd["model.encoder.embed_tokens.weight"] = sd["model.shared.weight"]
    sd["model.decoder.embed_tokens.weight"] = sd["model.shared.weight"]
    sd["lm_head.weight"] = sd["model.shared.weight"]
    missing, unexpected = model.load_state_dict(sd, strict=False)
    missing = [m for m in missing if "embed_positions" not in m]
    assert not missing and not unexpected, (missing, unexpected)
    s = max(len(r) for r in src)
    ids = torch.full((len(src), s), 1, dtype=torch.long)
    mask = torch.zeros((len(src), s), dtype=torch.long)
    for i, r in enumerate(src):
        ids[i, : len(r)] = torch.tensor(r)
        mask[i, : len(r)] = 1
    with torch.no_grad():
        out = model(input_ids=ids, attention_mask=mask, decoder_input_ids=torch.from_numpy(tgt.astype(np.int64)))
        enc = model.model.encoder(input_ids=ids, attention_mask=mask).last_hidden_state
    return out.logits.float().numpy(), enc.float().numpy()


def hf_greedy(weights: dict, src: list[list[int]], tgt_lang: int, max_new: int) -> np.ndarray:
    """transformers' greedy search with the target language forced as the first token
    (decoder_start = eos, src/translator.rs:214-241); no forced EOS, no length limits
    other than max_new greedy tokens after the language token."""
    from transformers import GenerationConfig, M2M100Config, M2M100ForConditionalGeneration

    cfg = M2M100Config(vocab_size=V, d_model=D, encoder_layers=LAYERS, decoder_layers=LAYERS,
                       encoder_attention_heads=H, decoder_attention_heads=H, encoder_ffn_dim=FFN,
                       decoder_ffn_dim=FFN, max_position_embeddings=MAXPOS, scale_embedding=True,
                       activation_function="relu", dropout=0.0, attention_dropout=0.0, activation_dropout=0.0,
                       encoder_layerdrop=0.0, decoder_layerdrop=0.0, pad_token_id=1, bos_token_id=0,
                       eos_token_id=2, decoder_start_token_id=2, tie_word_embeddings=True)
    cfg._attn_implementation = "eager"
    model = M2M100ForConditionalGeneration(cfg).eval()
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in weights.items()}
    for k in ("model.encoder.embed_tokens.weight", "model.decoder.embed_tokens.weight", "lm_head.weight"):
        sd[k] = sd["model.shared.weight"]
    model.load_state_dict(sd, strict=False)
    gen = GenerationConfig(decoder_start_token_id=2, forced_bos_token_id=tgt_lang, forced_eos_token_id=None,
                           eos_token_id=2, pad_token_id=1, bos_token_id=0, num_beams=1, do_sample=False,
                           max_new_tokens=max_new + 1, min_length=0)
    out = np.full((len(src), max_new), -1, dtype=np.int64)
    with torch.no_grad():
        for i, r in enumerate(src):  # one sentence at a time: no padding involved
            seq = model.generate(input_ids=torch.tensor([r]), generation_config=gen)[0].tolist()
            assert seq[:2] == [2, tgt_lang], seq[:2]
            toks = []
            for t in seq[2:]:
                if t == 2:
                    break
                toks.append(t)
            out[i, : len(toks)] = toks
    return out


def main():
    rng = np.random.default_rng(1234)
    # [src_lang] tokens [eos] (src/translator.rs:90-98) with the tiny vocabulary:
    # words 4..253, languages 254..256 (fra, eng, plt)
    src = [[254] + rng.integers(4, 254, size=n).tolist() + [2] for n in (9, 4, 13)]
    T = 12
    tgt = np.zeros((len(src), T), dtype=np.int64)
    tgt[:, 0] = 2      # decoder_start_token_id
    tgt[:, 1] = 256    # target language (plt_Latn)
    tgt[:, 2:] = rng.integers(4, 254, size=(len(src), T - 2))
    w = tiny_weights(7)
    logits, enc = hf_logits(w, src, tgt)
    wq = {k: (q8_0_roundtrip(v) if v.ndim == 2 else v) for k, v in w.items()}
    logits_q8, _ = hf_logits(wq, src, tgt)
    draw = xorshift_stream(7)
    first = draw(8, 0.5)
    lens = np.array([len(r) for r in src], dtype=np.uint32)
    ids = np.array([t for r in src for t in r], dtype=np.uint32)
    np.savez_compressed(OUT, src_ids=ids, src_lens=lens, tgt=tgt.astype(np.uint32), logits_f32=logits,
                        logits_q8_0=logits_q8, encoder_out=enc, xorshift_seed7_scale05=first,
                        greedy_255_20=hf_greedy(w, src, 255, 20), greedy_256_20=hf_greedy(w, src, 256, 20))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes); logits {logits.shape}, |logits| max {np.abs(logits).max():.3f}")


if __name__ == "__main__":
    main()
