#include "convert.hpp"

#include <algorithm>

#include <cmath>
#include <cstring>
#include <map>
#include <memory>

#include "gguf.hpp"
#include "quant.hpp"

namespace mlg {

bool preset_from_name(const std::string &s0, Preset *out) {
    std::string s;
    for (char c : s0) s.push_back(char(std::tolower(static_cast<unsigned char>(c))));
    static const std::pair<const char *, Preset> names[] = {{"f32", PRESET_F32},   {"f16", PRESET_F16},
                                                            {"q8_0", PRESET_Q8_0}, {"q6_k", PRESET_Q6K},
                                                            {"q5_k_m", PRESET_Q5KM}, {"q4_k_m", PRESET_Q4KM}};
    for (auto &n : names)
        if (s == n.first) { *out = n.second; return true; }
    return false;
}

const char *preset_name(Preset p) {
    switch (p) {
    case PRESET_F32: return "f32";
    case PRESET_F16: return "f16";
    case PRESET_Q8_0: return "q8_0";
    case PRESET_Q6K: return "q6_k";
    case PRESET_Q5KM: return "q5_k_m";
    case PRESET_Q4KM: return "q4_k_m";
    }
    return "?";
}

uint32_t preset_linear(Preset p) {
    switch (p) {
    case PRESET_F32: return GGML_F32;
    case PRESET_F16: return GGML_F16;
    case PRESET_Q8_0: return GGML_Q8_0;
    case PRESET_Q6K: return GGML_Q6_K;
    case PRESET_Q5KM: return GGML_Q5_K;
    case PRESET_Q4KM: return GGML_Q4_K;
    }
    return GGML_F32;
}

// The _m presets keep ffn_down and the embedding at Q6_K (src/convert.rs:78-91).
uint32_t preset_ffn_down(Preset p) { return (p == PRESET_Q5KM || p == PRESET_Q4KM) ? uint32_t(GGML_Q6_K) : preset_linear(p); }
uint32_t preset_embedding(Preset p) { return preset_ffn_down(p); }

uint32_t fallback_dtype(uint32_t dtype, const std::vector<int64_t> &dims) {
    if (dims.size() < 2) return GGML_F32;
    const int64_t row = dims.back();
    TypeInfo ti;
    type_info(dtype, &ti);
    if (row % ti.block_elems == 0) return dtype;
    if (row % 32 == 0) return GGML_Q8_0;
    return GGML_F16;
}

namespace {

struct Writer {
    std::vector<GgufOutTensor> tensors;
    std::string err;

    void add(const std::string &name, const std::vector<int64_t> &dims, const std::vector<float> &data, uint32_t dtype) {
        if (!err.empty()) return;
        dtype = fallback_dtype(dtype, dims);
        const int64_t k = dims.back();
        const int64_t rows = int64_t(data.size()) / k;
        GgufOutTensor t;
        t.name = name;
        for (auto it = dims.rbegin(); it != dims.rend(); ++it) t.ne.push_back(uint64_t(*it));
        t.type = dtype;
        t.bytes.resize(size_t(type_bytes(dtype, k) * rows));
        if (!quantize_rows(dtype, data.data(), rows, k, t.bytes.data())) err = "quantizing " + name;
        tensors.push_back(std::move(t));
    }
};

}  // namespace

std::string convert_to_gguf(const std::string &out_path, const ModelConfig &c, Preset preset,
                            const std::string &model_name, const std::string &tokenizer_json, const HfProvider &src,
                            const std::vector<ShortlistSpec> &shortlists) {
    if (c.d_model <= 0 || c.encoder_heads <= 0 || c.decoder_heads <= 0 || c.d_model % c.encoder_heads ||
        c.d_model % c.decoder_heads || c.vocab_size <= 0)
        return "invalid model config";
    const int64_t d = c.d_model;
    Writer w;
    std::string missing;
    auto take = [&](const std::string &name, int64_t numel) {
        std::vector<float> v(static_cast<size_t>(numel));
        if (missing.empty() && !src(name, numel, v.data())) missing = name;
        return v;
    };
    auto cat = [](std::vector<std::vector<float>> parts) {
        std::vector<float> o;
        for (auto &p : parts) o.insert(o.end(), p.begin(), p.end());
        return o;
    };
    auto scaled = [](std::vector<float> v, float s) {
        for (auto &x : v) x = x * s;
        return v;
    };

    w.add("token_embd.weight", {c.vocab_size, d}, take("model.shared.weight", int64_t(c.vocab_size) * d),
          preset_embedding(preset));
    // src/convert.rs:218-233: per-language shortlists.  Quantization is row-local, so the
    // rows of the shared table quantized for lm_head.{code} are token_embd's own rows:
    // they are copied.
    std::vector<std::pair<std::string, GgufValue>> sl_meta;
    for (const ShortlistSpec &sl : shortlists) {
        if (!w.err.empty() || !missing.empty()) break;
        if (sl.code.empty()) return "shortlist without a language code";
        std::vector<uint32_t> ids = {0, 1, 2, 3, sl.lang_id};
        for (uint32_t id : sl.ids)
            if (id < uint32_t(c.vocab_size)) ids.push_back(id);
        std::sort(ids.begin(), ids.end());
        ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
        if (ids.back() >= uint32_t(c.vocab_size)) return "shortlist language id out of range";
        const GgufOutTensor &emb = w.tensors.front();
        const size_t rb = size_t(type_bytes(emb.type, d));
        GgufOutTensor t;
        t.name = "lm_head." + sl.code + ".weight";
        t.ne = {uint64_t(d), uint64_t(ids.size())};
        t.type = emb.type;
        t.bytes.resize(rb * ids.size());
        for (size_t r = 0; r < ids.size(); ++r)
            std::memcpy(t.bytes.data() + r * rb, emb.bytes.data() + size_t(ids[r]) * rb, rb);
        w.tensors.push_back(std::move(t));
        sl_meta.push_back({"nllb.shortlist." + sl.code, GgufValue::ArrU32(ids)});
    }
    const uint32_t lin = preset_linear(preset), down = preset_ffn_down(preset);
    for (int side = 0; side < 2; ++side) {
        const bool dec = side == 1;
        const std::string sname = dec ? "decoder" : "encoder", sh = dec ? "dec" : "enc";
        const int layers = dec ? c.decoder_layers : c.encoder_layers;
        const int64_t ffn = dec ? c.decoder_ffn : c.encoder_ffn;
        const int heads = dec ? c.decoder_heads : c.encoder_heads;
        // 1/sqrt(head_dim) folded into the query weights and bias (src/convert.rs:211-212, 243-244, 258-259)
        const float s = float(std::pow(double(d / heads), -0.5));
        for (int i = 0; i < layers; ++i) {
            const std::string p = "model." + sname + ".layers." + std::to_string(i), o = sh + ".blk." + std::to_string(i);
            auto qkv_w = cat({scaled(take(p + ".self_attn.q_proj.weight", d * d), s), take(p + ".self_attn.k_proj.weight", d * d),
                              take(p + ".self_attn.v_proj.weight", d * d)});
            auto qkv_b = cat({scaled(take(p + ".self_attn.q_proj.bias", d), s), take(p + ".self_attn.k_proj.bias", d),
                              take(p + ".self_attn.v_proj.bias", d)});
            w.add(o + ".attn_qkv.weight", {3 * d, d}, qkv_w, lin);
            w.add(o + ".attn_qkv.bias", {3 * d}, qkv_b, GGML_F32);
            w.add(o + ".attn_out.weight", {d, d}, take(p + ".self_attn.out_proj.weight", d * d), lin);
            w.add(o + ".attn_out.bias", {d}, take(p + ".self_attn.out_proj.bias", d), GGML_F32);
            w.add(o + ".attn_norm.weight", {d}, take(p + ".self_attn_layer_norm.weight", d), GGML_F32);
            w.add(o + ".attn_norm.bias", {d}, take(p + ".self_attn_layer_norm.bias", d), GGML_F32);
            if (dec) {
                w.add(o + ".cross_attn_q.weight", {d, d}, scaled(take(p + ".encoder_attn.q_proj.weight", d * d), s), lin);
                w.add(o + ".cross_attn_q.bias", {d}, scaled(take(p + ".encoder_attn.q_proj.bias", d), s), GGML_F32);
                w.add(o + ".cross_attn_kv.weight", {2 * d, d},
                      cat({take(p + ".encoder_attn.k_proj.weight", d * d), take(p + ".encoder_attn.v_proj.weight", d * d)}), lin);
                w.add(o + ".cross_attn_kv.bias", {2 * d},
                      cat({take(p + ".encoder_attn.k_proj.bias", d), take(p + ".encoder_attn.v_proj.bias", d)}), GGML_F32);
                w.add(o + ".cross_attn_out.weight", {d, d}, take(p + ".encoder_attn.out_proj.weight", d * d), lin);
                w.add(o + ".cross_attn_out.bias", {d}, take(p + ".encoder_attn.out_proj.bias", d), GGML_F32);
                w.add(o + ".cross_attn_norm.weight", {d}, take(p + ".encoder_attn_layer_norm.weight", d), GGML_F32);
                w.add(o + ".cross_attn_norm.bias", {d}, take(p + ".encoder_attn_layer_norm.bias", d), GGML_F32);
            }
            w.add(o + ".ffn_up.weight", {ffn, d}, take(p + ".fc1.weight", ffn * d), lin);
            w.add(o + ".ffn_up.bias", {ffn}, take(p + ".fc1.bias", ffn), GGML_F32);
            w.add(o + ".ffn_down.weight", {d, ffn}, take(p + ".fc2.weight", d * ffn), down);
            w.add(o + ".ffn_down.bias", {d}, take(p + ".fc2.bias", d), GGML_F32);
            w.add(o + ".ffn_norm.weight", {d}, take(p + ".final_layer_norm.weight", d), GGML_F32);
            w.add(o + ".ffn_norm.bias", {d}, take(p + ".final_layer_norm.bias", d), GGML_F32);
            if (!missing.empty()) return "missing tensor " + missing;
        }
        w.add(sh + ".output_norm.weight", {d}, take("model." + sname + ".layer_norm.weight", d), GGML_F32);
        w.add(sh + ".output_norm.bias", {d}, take("model." + sname + ".layer_norm.bias", d), GGML_F32);
    }
    if (!missing.empty()) return "missing tensor " + missing;
    if (!w.err.empty()) return w.err;

    // src/convert.rs:293-303 and src/config.rs:71-91
    std::vector<std::pair<std::string, GgufValue>> kv = {
        {"general.architecture", GgufValue::Str("nllb")},
        {"general.name", GgufValue::Str(model_name)},
        {"general.file_type", GgufValue::Str(preset_name(preset))},
        {"general.license", GgufValue::Str("cc-by-nc-4.0")},
        {"general.source.url", GgufValue::Str("https://huggingface.co/" + model_name)},
        {"tokenizer.ggml.model", GgufValue::Str("nllb")},
        {"tokenizer.huggingface.json", GgufValue::Str(tokenizer_json)},
        {"nllb.vocab_size", GgufValue::U32(uint32_t(c.vocab_size))},
        {"nllb.embedding_length", GgufValue::U32(uint32_t(c.d_model))},
        {"nllb.encoder.block_count", GgufValue::U32(uint32_t(c.encoder_layers))},
        {"nllb.decoder.block_count", GgufValue::U32(uint32_t(c.decoder_layers))},
        {"nllb.encoder.attention.head_count", GgufValue::U32(uint32_t(c.encoder_heads))},
        {"nllb.decoder.attention.head_count", GgufValue::U32(uint32_t(c.decoder_heads))},
        {"nllb.encoder.feed_forward_length", GgufValue::U32(uint32_t(c.encoder_ffn))},
        {"nllb.decoder.feed_forward_length", GgufValue::U32(uint32_t(c.decoder_ffn))},
        {"nllb.context_length", GgufValue::U32(uint32_t(c.max_position_embeddings))},
        {"nllb.scale_embedding", GgufValue::Bool(c.scale_embedding != 0)},
        {"nllb.max_length", GgufValue::U32(uint32_t(c.max_length))},
        {"tokenizer.ggml.bos_token_id", GgufValue::U32(uint32_t(c.bos_token_id))},
        {"tokenizer.ggml.padding_token_id", GgufValue::U32(uint32_t(c.pad_token_id))},
        {"tokenizer.ggml.eos_token_id", GgufValue::U32(uint32_t(c.eos_token_id))},
        {"tokenizer.ggml.decoder_start_token_id", GgufValue::U32(uint32_t(c.decoder_start_token_id))},
    };
    kv.insert(kv.end(), sl_meta.begin(), sl_meta.end());
    return gguf_write(out_path, kv, w.tensors);
}

namespace {

inline uint64_t splitmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t fnv1a(const std::string &s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char ch : s) h = (h ^ ch) * 0x100000001b3ull;
    return h;
}

// Element i of a counter-based N(0,1) stream: Box-Muller on two splitmix64 draws
// per pair (cosine for even i, sine for odd i).
void normal_fill(uint64_t key, int64_t n, float std_dev, float mean, float *out) {
    const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < (n + 1) / 2; ++p) {
        const uint64_t r1 = splitmix64(key + uint64_t(2 * p + 1) * 0x9E3779B97F4A7C15ull);
        const uint64_t r2 = splitmix64(key + uint64_t(2 * p + 2) * 0x9E3779B97F4A7C15ull);
        const double u1 = (double((r1 >> 11) + 1)) * (1.0 / 9007199254740992.0);  // (0, 1]
        const double u2 = double(r2 >> 11) * (1.0 / 9007199254740992.0);          // [0, 1)
        const double rad = std::sqrt(-2.0 * std::log(u1));
        out[2 * p] = float(mean + std_dev * rad * std::cos(two_pi * u2));
        if (2 * p + 1 < n) out[2 * p + 1] = float(mean + std_dev * rad * std::sin(two_pi * u2));
    }
}

bool ends_with(const std::string &s, const std::string &suf) {
    return s.size() >= suf.size() && s.compare(s.size() - suf.size(), suf.size(), suf) == 0;
}

}  // namespace

HfProvider synthetic_provider(const ModelConfig &c, SynthInit init, uint64_t seed, float std_dev) {
    if (init == SYNTH_TESTUTIL) {
        // src/testutil.rs:56-99, same draw order as the reference's insertion order.
        auto tensors = std::make_shared<std::map<std::string, std::vector<float>>>();
        uint64_t state = (seed * 0x9E3779B97F4A7C15ull) | 1;
        auto rnd = [&](const std::string &name, int64_t n, float scale) {
            std::vector<float> v(static_cast<size_t>(n));
            for (auto &x : v) {
                state ^= state << 13;
                state ^= state >> 7;
                state ^= state << 17;
                x = (float(state >> 40) / float(1u << 24) - 0.5f) * 2.0f * scale;
            }
            (*tensors)[name] = std::move(v);
        };
        const int64_t d = c.d_model;
        rnd("model.shared.weight", int64_t(c.vocab_size) * d, 0.5f);
        for (int side = 0; side < 2; ++side) {
            const std::string sn = side ? "decoder" : "encoder";
            const int layers = side ? c.decoder_layers : c.encoder_layers;
            const int64_t ffn = side ? c.decoder_ffn : c.encoder_ffn;
            for (int l = 0; l < layers; ++l) {
                const std::string p = "model." + sn + ".layers." + std::to_string(l);
                std::vector<std::string> attns = {"self_attn"};
                if (side) attns.push_back("encoder_attn");
                for (auto &a : attns) {
                    for (const char *proj : {"q_proj", "k_proj", "v_proj", "out_proj"}) {
                        rnd(p + "." + a + "." + proj + ".weight", d * d, 0.3f);
                        rnd(p + "." + a + "." + proj + ".bias", d, 0.1f);
                    }
                    (*tensors)[p + "." + a + "_layer_norm.weight"] = std::vector<float>(size_t(d), 1.f);
                    (*tensors)[p + "." + a + "_layer_norm.bias"] = std::vector<float>(size_t(d), 0.f);
                }
                rnd(p + ".fc1.weight", ffn * d, 0.3f);
                rnd(p + ".fc1.bias", ffn, 0.1f);
                rnd(p + ".fc2.weight", d * ffn, 0.3f);
                rnd(p + ".fc2.bias", d, 0.1f);
                (*tensors)[p + ".final_layer_norm.weight"] = std::vector<float>(size_t(d), 1.f);
                (*tensors)[p + ".final_layer_norm.bias"] = std::vector<float>(size_t(d), 0.f);
            }
            (*tensors)["model." + sn + ".layer_norm.weight"] = std::vector<float>(size_t(d), 1.f);
            (*tensors)["model." + sn + ".layer_norm.bias"] = std::vector<float>(size_t(d), 0.f);
        }
        return [tensors](const std::string &name, int64_t n, float *out) {
            auto it = tensors->find(name);
            if (it == tensors->end() || int64_t(it->second.size()) != n) return false;
            std::memcpy(out, it->second.data(), size_t(n) * 4);
            return true;
        };
    }
    const bool rich = init == SYNTH_NORMAL_RICH;
    const int pad = c.pad_token_id, d = c.d_model;
    return [=](const std::string &name, int64_t n, float *out) {
        const uint64_t key = splitmix64(fnv1a(name) ^ (seed * 0xD1B54A32D192ED03ull));
        const bool norm = name.find("layer_norm") != std::string::npos;
        if (norm) {
            const bool gamma = ends_with(name, ".weight");
            if (rich) normal_fill(key, n, 0.1f, gamma ? 1.f : 0.f, out);
            else for (int64_t i = 0; i < n; ++i) out[i] = gamma ? 1.f : 0.f;
        } else if (ends_with(name, ".bias")) {
            if (rich) normal_fill(key, n, 0.05f, 0.f, out);
            else std::memset(out, 0, size_t(n) * 4);
        } else {
            normal_fill(key, n, std_dev, 0.f, out);
            if (name == "model.shared.weight" && int64_t(pad + 1) * d <= n) std::memset(out + int64_t(pad) * d, 0, size_t(d) * 4);
        }
        return true;
    };
}

std::string tiny_tokenizer_json(int vocab_size) {
    // src/testutil.rs:33-54: <s> <pad> </s> <unk>, words w0.., then the language codes.
    static const char *specials[] = {"<s>", "<pad>", "</s>", "<unk>"};
    static const char *langs[] = {"fra_Latn", "eng_Latn", "plt_Latn"};
    const int words = vocab_size - 4 - 3;
    std::string vocab, added;
    for (int i = 0; i < 4; ++i) {
        vocab += std::string(i ? "," : "") + "\"" + specials[i] + "\":" + std::to_string(i);
        added += std::string(i ? "," : "") + "{\"id\":" + std::to_string(i) + ",\"content\":\"" + specials[i] +
                 "\",\"single_word\":false,\"lstrip\":false,\"rstrip\":false,\"normalized\":false,\"special\":true}";
    }
    for (int w = 0; w < words; ++w) vocab += ",\"w" + std::to_string(w) + "\":" + std::to_string(4 + w);
    for (int i = 0; i < 3; ++i) {
        const int id = 4 + words + i;
        vocab += std::string(",\"") + langs[i] + "\":" + std::to_string(id);
        added += ",{\"id\":" + std::to_string(id) + ",\"content\":\"" + langs[i] +
                 "\",\"single_word\":false,\"lstrip\":false,\"rstrip\":false,\"normalized\":false,\"special\":true}";
    }
    return "{\"version\":\"1.0\",\"truncation\":null,\"padding\":null,\"added_tokens\":[" + added +
           "],\"normalizer\":null,\"pre_tokenizer\":{\"type\":\"Whitespace\"},\"post_processor\":null,"
           "\"decoder\":null,\"model\":{\"type\":\"WordLevel\",\"vocab\":{" + vocab + "},\"unk_token\":\"<unk>\"}}";
}

}  // namespace mlg
