// Hugging Face NLLB checkpoint -> GGUF conversion (src/convert.rs), plus the
// synthetic checkpoints used by tests and benchmarks.
#pragma once
#include <cstdint>
#include <functional>
#include <string>
#include <vector>

namespace mlg {

// src/config.rs:14-39 (hyper-parameters of an NLLB / M2M100 checkpoint)
struct ModelConfig {
    int vocab_size = 0, d_model = 0, encoder_layers = 0, decoder_layers = 0;
    int encoder_heads = 0, decoder_heads = 0, encoder_ffn = 0, decoder_ffn = 0;
    int max_position_embeddings = 0, max_length = 200, scale_embedding = 1;
    int bos_token_id = 0, pad_token_id = 1, eos_token_id = 2, decoder_start_token_id = 2;
};

// src/convert.rs:25-91
enum Preset : int { PRESET_F32 = 0, PRESET_F16, PRESET_Q8_0, PRESET_Q6K, PRESET_Q5KM, PRESET_Q4KM };
bool preset_from_name(const std::string &s, Preset *out);
const char *preset_name(Preset p);
uint32_t preset_linear(Preset p);
uint32_t preset_ffn_down(Preset p);
uint32_t preset_embedding(Preset p);
// src/convert.rs:148-162: k-quants need rows % 256, legacy quants rows % 32.
uint32_t fallback_dtype(uint32_t dtype, const std::vector<int64_t> &dims);

// Supplies the f32 data of a Hugging Face tensor by name ("model.shared.weight",
// "model.encoder.layers.0.self_attn.q_proj.weight", ...).  The expected element
// count is passed in; return false if the tensor is missing.
using HfProvider = std::function<bool(const std::string &name, int64_t numel, float *out)>;

// A reduced LM head for one target language (src/convert.rs:176-233): the vocabulary
// ids a corpus of that language uses.  The writer adds <s> <pad> </s> <unk> (ids 0..3)
// and the language token, sorts, and stores the rows of token_embd for those ids as
// lm_head.{code}.weight plus the id list as nllb.shortlist.{code}.  (The reference
// derives `ids` by tokenizing a corpus; here the caller passes them.)
struct ShortlistSpec {
    std::string code;
    uint32_t lang_id = 0;
    std::vector<uint32_t> ids;
};

// src/convert.rs:196-318.  Returns "" on success.
std::string convert_to_gguf(const std::string &out_path, const ModelConfig &cfg, Preset preset,
                            const std::string &model_name, const std::string &tokenizer_json, const HfProvider &src,
                            const std::vector<ShortlistSpec> &shortlists = {});

// Synthetic checkpoints.
enum SynthInit : int {
    // src/testutil.rs:56-99: xorshift64 weights (embedding 0.5, projections 0.3,
    // biases 0.1), LayerNorm gamma 1 / beta 0.  Tensors drawn in testutil's order.
    SYNTH_TESTUTIL = 0,
    // Random init of the benchmark models: rank >= 2 tensors ~ N(0, std), biases 0,
    // LayerNorm 1/0, embedding row `pad` zeroed.  splitmix64 + Box-Muller, counter based.
    SYNTH_NORMAL = 1,
    // Parity fixture: N(0, std) weights plus non-zero biases ~ N(0, 0.05) and
    // LayerNorm gamma ~ 1 + N(0, 0.1), beta ~ N(0, 0.1), so every term is exercised.
    SYNTH_NORMAL_RICH = 2,
};
HfProvider synthetic_provider(const ModelConfig &cfg, SynthInit init, uint64_t seed, float std_dev);

// Tokenizer JSON of the tiny test vocabulary (src/testutil.rs:33-54).
std::string tiny_tokenizer_json(int vocab_size);

}  // namespace mlg
