"""GGUF layout written by the converter (src/convert.rs:196-318, src/config.rs:71-91)."""
import numpy as np
import pytest

import malaga_amd as M
from tests.conftest import KQ_CONFIG
from malaga_amd.gguf import read_gguf

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 8, 12, 13, 14


def test_metadata_keys(tiny_gguf):
    version, meta, tensors, _ = read_gguf(tiny_gguf("q8_0"))
    assert version == 3
    assert meta["general.architecture"] == "nllb"
    assert meta["general.file_type"] == "q8_0"
    cfg = M.tiny_config()
    assert meta["nllb.vocab_size"] == cfg["vocab_size"] == 257
    assert meta["nllb.embedding_length"] == 64
    assert meta["nllb.encoder.block_count"] == meta["nllb.decoder.block_count"] == 2
    assert meta["nllb.decoder.attention.head_count"] == 4
    assert meta["nllb.decoder.feed_forward_length"] == 128
    assert meta["nllb.context_length"] == 128 and meta["nllb.max_length"] == 64
    assert meta["nllb.scale_embedding"] is True
    assert (meta["tokenizer.ggml.padding_token_id"], meta["tokenizer.ggml.eos_token_id"],
            meta["tokenizer.ggml.decoder_start_token_id"], meta["tokenizer.ggml.bos_token_id"]) == (1, 2, 2, 0)
    assert '"WordLevel"' in meta["tokenizer.huggingface.json"]


def test_tensor_names_and_shapes(tiny_gguf):
    _, _, tensors, _ = read_gguf(tiny_gguf("f32"))
    d, f = 64, 128
    want = {"token_embd.weight": [d, 257], "enc.output_norm.weight": [d], "dec.output_norm.bias": [d]}
    for side in ("enc", "dec"):
        for i in range(2):
            p = f"{side}.blk.{i}"
            want[f"{p}.attn_qkv.weight"] = [d, 3 * d]
            want[f"{p}.attn_qkv.bias"] = [3 * d]
            want[f"{p}.attn_out.weight"] = [d, d]
            want[f"{p}.ffn_up.weight"] = [d, f]
            want[f"{p}.ffn_down.weight"] = [f, d]
            want[f"{p}.ffn_norm.weight"] = [d]
            if side == "dec":
                want[f"{p}.cross_attn_q.weight"] = [d, d]
                want[f"{p}.cross_attn_kv.weight"] = [d, 2 * d]
                want[f"{p}.cross_attn_out.bias"] = [d]
                want[f"{p}.cross_attn_norm.weight"] = [d]
    for name, ne in want.items():
        assert tensors[name]["ne"] == ne, name
    assert not any(n.startswith("lm_head") for n in tensors)  # tied LM head (src/model.rs:312-313)


def test_tiny_q4_k_m_falls_back_to_q8_0(tiny_gguf):
    """Rows of 64/128 values are not a multiple of 256: k-quants fall back (src/convert.rs:148-162)."""
    _, _, tensors, _ = read_gguf(tiny_gguf("q4_k_m"))
    assert tensors["dec.blk.0.attn_qkv.weight"]["type"] == Q8_0
    assert tensors["dec.blk.0.ffn_down.weight"]["type"] == Q8_0
    assert tensors["token_embd.weight"]["type"] == Q8_0
    assert tensors["dec.blk.0.attn_qkv.bias"]["type"] == F32
    assert tensors["dec.blk.0.ffn_norm.weight"]["type"] == F32


@pytest.mark.parametrize("preset,lin,down,emb", [("q4_k_m", Q4_K, Q6_K, Q6_K), ("q5_k_m", Q5_K, Q6_K, Q6_K),
                                                 ("q6_k", Q6_K, Q6_K, Q6_K), ("q8_0", Q8_0, Q8_0, Q8_0),
                                                 ("f16", F16, F16, F16)])
def test_preset_type_map(kq_gguf, preset, lin, down, emb):
    """src/convert.rs:78-91: _m presets keep ffn_down and the embedding at Q6_K."""
    _, _, tensors, _ = read_gguf(kq_gguf(preset))
    for name in ("attn_qkv", "attn_out", "ffn_up", "cross_attn_q", "cross_attn_kv", "cross_attn_out"):
        assert tensors[f"dec.blk.1.{name}.weight"]["type"] == lin, name
    assert tensors["enc.blk.0.ffn_down.weight"]["type"] == down
    assert tensors["token_embd.weight"]["type"] == emb
    assert tensors["enc.blk.0.attn_norm.bias"]["type"] == F32


def test_fused_qkv_order_and_query_prescale(tmp_path):
    """attn_qkv = cat(q * hd^-0.5, k, v) (src/convert.rs:242-251, 258-267); cross q pre-scaled, kv = cat(k, v)."""
    cfg = dict(M.tiny_config())
    rng = np.random.default_rng(0)
    d, f, V = cfg["d_model"], cfg["encoder_ffn"], cfg["vocab_size"]
    w = {"model.shared.weight": rng.normal(0, 1, (V, d))}
    for side in ("encoder", "decoder"):
        for l in range(2):
            p = f"model.{side}.layers.{l}"
            for a in ["self_attn"] + (["encoder_attn"] if side == "decoder" else []):
                for proj in ("q_proj", "k_proj", "v_proj", "out_proj"):
                    w[f"{p}.{a}.{proj}.weight"] = rng.normal(0, 1, (d, d))
                    w[f"{p}.{a}.{proj}.bias"] = rng.normal(0, 1, d)
                w[f"{p}.{a}_layer_norm.weight"] = np.ones(d)
                w[f"{p}.{a}_layer_norm.bias"] = np.zeros(d)
            w[f"{p}.fc1.weight"], w[f"{p}.fc1.bias"] = rng.normal(0, 1, (f, d)), rng.normal(0, 1, f)
            w[f"{p}.fc2.weight"], w[f"{p}.fc2.bias"] = rng.normal(0, 1, (d, f)), rng.normal(0, 1, d)
            w[f"{p}.final_layer_norm.weight"], w[f"{p}.final_layer_norm.bias"] = np.ones(d), np.zeros(d)
        w[f"model.{side}.layer_norm.weight"], w[f"model.{side}.layer_norm.bias"] = np.ones(d), np.zeros(d)
    w = {k: v.astype(np.float32) for k, v in w.items()}
    out = M.convert(tmp_path / "c.gguf", cfg, "f32", w)
    _, _, tensors, data = read_gguf(out)

    def get(name, shape):
        t = tensors[name]
        return np.frombuffer(data, np.float32, count=int(np.prod(shape)), offset=t["data_start"]).reshape(shape)

    s = np.float32((d // cfg["decoder_heads"]) ** -0.5)
    qkv = get("dec.blk.1.attn_qkv.weight", (3 * d, d))
    p = "model.decoder.layers.1.self_attn"
    np.testing.assert_array_equal(qkv[:d], w[f"{p}.q_proj.weight"] * s)
    np.testing.assert_array_equal(qkv[d:2 * d], w[f"{p}.k_proj.weight"])
    np.testing.assert_array_equal(qkv[2 * d:], w[f"{p}.v_proj.weight"])
    b = get("dec.blk.1.attn_qkv.bias", (3 * d,))
    np.testing.assert_array_equal(b[:d], w[f"{p}.q_proj.bias"] * s)
    cq = get("dec.blk.0.cross_attn_q.bias", (d,))
    np.testing.assert_array_equal(cq, w["model.decoder.layers.0.encoder_attn.q_proj.bias"] * s)
    kv = get("dec.blk.0.cross_attn_kv.weight", (2 * d, d))
    np.testing.assert_array_equal(kv[d:], w["model.decoder.layers.0.encoder_attn.v_proj.weight"])


def test_missing_tensor_is_an_error(tmp_path):
    with pytest.raises(M.MalagaError, match="missing tensor"):
        M.convert(tmp_path / "x.gguf", M.tiny_config(), "f32", {})


def test_synthetic_normal_init(tmp_path):
    """Benchmark init: rank-2 ~ N(0, std), biases 0, LN 1/0, pad row zeroed; deterministic."""
    cfg = dict(KQ_CONFIG)
    a = M.write_synthetic(tmp_path / "a.gguf", cfg, "f32", M.INIT_NORMAL, seed=0, std=0.02)
    b = M.write_synthetic(tmp_path / "b.gguf", cfg, "f32", M.INIT_NORMAL, seed=0, std=0.02)
    assert a.read_bytes() == b.read_bytes()
    _, _, tensors, data = read_gguf(a)
    t = tensors["token_embd.weight"]
    e = np.frombuffer(data, np.float32, count=1000 * 256, offset=t["data_start"]).reshape(1000, 256)
    assert (e[1] == 0).all()
    assert abs(e.std() - 0.02) < 5e-4 and abs(e.mean()) < 5e-4
    bias = np.frombuffer(data, np.float32, count=768, offset=tensors["dec.blk.0.attn_qkv.bias"]["data_start"])
    assert (bias == 0).all()
