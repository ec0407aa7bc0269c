// extern "C" layer of libmalaga_hip.so (declarations and reference citations in
// include/malaga_hip.h).  Translates exceptions into status codes + a
// thread-local message.
#include "../../include/malaga_hip.h"

#include <cstring>
#include <initializer_list>
#include <memory>
#include <string>

#include "beam.hpp"
#include "convert.hpp"
#include "quant.hpp"
#include "runtime.hpp"
#include "server.hpp"

struct mlg_ctx {
    mlg::Context c;
};
struct mlg_model {
    std::unique_ptr<mlg::Model> m;
};
struct mlg_batch {
    std::unique_ptr<mlg::Batch> b;
};
struct mlg_server {
    std::unique_ptr<mlg::Server> s;
};
struct mlg_job {
    std::shared_ptr<mlg::Job> j;
};
struct mlg_matrix {
    mlg::DevMatrix w;
    void *mem = nullptr;
    void *mem_lm = nullptr;
    void *mem_tm = nullptr;
    ~mlg_matrix() {
        mlg::dev_free(mem);
        mlg::dev_free(mem_lm);
        mlg::dev_free(mem_tm);
    }
    mlg_ctx *ctx = nullptr;
};

namespace {

thread_local std::string g_last_error;

int set_err(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

template <typename F>
int guarded(F &&f) {
    try {
        g_last_error.clear();
        return f();
    } catch (const mlg::Failure &e) {
        return set_err(e.code, e.msg);
    } catch (const std::bad_alloc &) {
        return set_err(MLG_ERR_OOM, "OUT_OF_MEMORY: host allocation failed");
    } catch (const std::exception &e) {
        return set_err(MLG_ERR_INVALID, e.what());
    }
}

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return MLG_OK;
    if (e == hipErrorOutOfMemory) return set_err(MLG_ERR_OOM, std::string("OUT_OF_MEMORY: ") + what);
    if (e == hipErrorInvalidValue) return set_err(MLG_ERR_INVALID, std::string(what) + ": invalid arguments");
    return set_err(MLG_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

mlg::ModelConfig to_cfg(const mlg_config *c) {
    mlg::ModelConfig m;
    m.vocab_size = c->vocab_size;
    m.d_model = c->d_model;
    m.encoder_layers = c->encoder_layers;
    m.decoder_layers = c->decoder_layers;
    m.encoder_heads = c->encoder_heads;
    m.decoder_heads = c->decoder_heads;
    m.encoder_ffn = c->encoder_ffn;
    m.decoder_ffn = c->decoder_ffn;
    m.max_position_embeddings = c->max_position_embeddings;
    m.max_length = c->max_length;
    m.scale_embedding = c->scale_embedding;
    m.bos_token_id = c->bos_token_id;
    m.pad_token_id = c->pad_token_id;
    m.eos_token_id = c->eos_token_id;
    m.decoder_start_token_id = c->decoder_start_token_id;
    return m;
}

void from_cfg(const mlg::ModelConfig &m, mlg_config *c) {
    c->vocab_size = m.vocab_size;
    c->d_model = m.d_model;
    c->encoder_layers = m.encoder_layers;
    c->decoder_layers = m.decoder_layers;
    c->encoder_heads = m.encoder_heads;
    c->decoder_heads = m.decoder_heads;
    c->encoder_ffn = m.encoder_ffn;
    c->decoder_ffn = m.decoder_ffn;
    c->max_position_embeddings = m.max_position_embeddings;
    c->max_length = m.max_length;
    c->scale_embedding = m.scale_embedding;
    c->bos_token_id = m.bos_token_id;
    c->pad_token_id = m.pad_token_id;
    c->eos_token_id = m.eos_token_id;
    c->decoder_start_token_id = m.decoder_start_token_id;
}

std::vector<std::vector<uint32_t>> rows_of(const uint32_t *ids, const uint32_t *lens, int n) {
    std::vector<std::vector<uint32_t>> src(size_t(n > 0 ? n : 0));
    size_t off = 0;
    for (int i = 0; i < n; ++i) {
        src[i].assign(ids + off, ids + off + lens[i]);
        off += lens[i];
    }
    return src;
}

bool aligned16(std::initializer_list<const void *> ptrs) {
    for (const void *p : ptrs)
        if (reinterpret_cast<uintptr_t>(p) % 16) return false;
    return true;
}

int write_rows(const std::vector<std::vector<uint32_t>> &rows, uint32_t *out, int out_cap, int *out_len) {
    for (size_t i = 0; i < rows.size(); ++i) {
        const int n = int(rows[i].size());
        if (n > out_cap) return set_err(MLG_ERR_INVALID, "output row longer than out_cap");
        if (n) std::memcpy(out + i * size_t(out_cap), rows[i].data(), size_t(n) * 4);
        out_len[i] = n;
    }
    return MLG_OK;
}

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

const char *mlg_last_error(void) { return g_last_error.c_str(); }
const char *mlg_version(void) { return "malaga_hip 0.1 (gfx950)"; }

int mlg_type_info(uint32_t type, int *block_elems, int *block_bytes) {
    mlg::TypeInfo ti;
    if (!mlg::type_info(type, &ti)) return set_err(MLG_ERR_UNSUPPORTED, "unsupported ggml type");
    *block_elems = ti.block_elems;
    *block_bytes = ti.block_bytes;
    return MLG_OK;
}

int64_t mlg_type_bytes(uint32_t type, int64_t n) { return mlg::type_bytes(type, n); }

int mlg_quantize(uint32_t type, const float *x, int64_t n, void *out) {
    return mlg::quantize(type, x, n, out) ? MLG_OK : set_err(MLG_ERR_INVALID, "quantize: bad type or length");
}

int mlg_dequantize(uint32_t type, const void *in, int64_t n, float *out) {
    return mlg::dequantize(type, in, n, out) ? MLG_OK : set_err(MLG_ERR_INVALID, "dequantize: bad type or length");
}

int mlg_preset_from_name(const char *name, int *preset) {
    mlg::Preset p;
    if (!name || !mlg::preset_from_name(name, &p))
        return set_err(MLG_ERR_INVALID, std::string("unknown preset '") + (name ? name : "") +
                                            "' (f32, f16, q8_0, q6_k, q5_k_m, q4_k_m)");
    *preset = int(p);
    return MLG_OK;
}

namespace {
bool to_shortlists(const mlg_shortlist_spec *sl, int n, std::vector<mlg::ShortlistSpec> *out) {
    if (n < 0 || (n > 0 && !sl)) return false;
    for (int i = 0; i < n; ++i) {
        if (!sl[i].code || sl[i].n_ids < 0 || (sl[i].n_ids > 0 && !sl[i].ids)) return false;
        mlg::ShortlistSpec t;
        t.code = sl[i].code;
        t.lang_id = sl[i].lang_id;
        t.ids.assign(sl[i].ids, sl[i].ids + sl[i].n_ids);
        out->push_back(std::move(t));
    }
    return true;
}
}  // namespace

int mlg_convert_sl(const char *out_path, const mlg_config *cfg, int preset, const char *model_name,
                   const char *tokenizer_json, mlg_tensor_fn fn, void *user, const mlg_shortlist_spec *sl, int n_sl) {
    return guarded([&]() -> int {
        if (preset < 0 || preset > mlg::PRESET_Q4KM) return set_err(MLG_ERR_INVALID, "unknown preset");
        std::vector<mlg::ShortlistSpec> lists;
        if (!to_shortlists(sl, n_sl, &lists)) return set_err(MLG_ERR_INVALID, "bad shortlist");
        auto src = [&](const std::string &name, int64_t n, float *out) { return fn(user, name.c_str(), n, out) == 0; };
        const std::string e = mlg::convert_to_gguf(out_path, to_cfg(cfg), mlg::Preset(preset), model_name ? model_name : "",
                                                   tokenizer_json ? tokenizer_json : "{}", src, lists);
        return e.empty() ? MLG_OK : set_err(MLG_ERR_IO, e);
    });
}

int mlg_convert(const char *out_path, const mlg_config *cfg, int preset, const char *model_name,
                const char *tokenizer_json, mlg_tensor_fn fn, void *user) {
    return mlg_convert_sl(out_path, cfg, preset, model_name, tokenizer_json, fn, user, nullptr, 0);
}

int mlg_write_synthetic_sl(const char *out_path, const mlg_config *cfg, int preset, int init, uint64_t seed,
                           float std_dev, const char *model_name, const mlg_shortlist_spec *sl, int n_sl) {
    return guarded([&]() -> int {
        if (preset < 0 || preset > mlg::PRESET_Q4KM) return set_err(MLG_ERR_INVALID, "unknown preset");
        if (init < 0 || init > 2) return set_err(MLG_ERR_INVALID, "unknown init");
        std::vector<mlg::ShortlistSpec> lists;
        if (!to_shortlists(sl, n_sl, &lists)) return set_err(MLG_ERR_INVALID, "bad shortlist");
        const mlg::ModelConfig c = to_cfg(cfg);
        auto src = mlg::synthetic_provider(c, mlg::SynthInit(init), seed, std_dev);
        const std::string tok = init == mlg::SYNTH_TESTUTIL ? mlg::tiny_tokenizer_json(c.vocab_size)
                                                            : std::string("{\"synthetic\":true}");
        const std::string e = mlg::convert_to_gguf(out_path, c, mlg::Preset(preset),
                                                   model_name ? model_name : "synthetic", tok, src, lists);
        return e.empty() ? MLG_OK : set_err(MLG_ERR_IO, e);
    });
}

int mlg_write_synthetic(const char *out_path, const mlg_config *cfg, int preset, int init, uint64_t seed,
                        float std_dev, const char *model_name) {
    return mlg_write_synthetic_sl(out_path, cfg, preset, init, seed, std_dev, model_name, nullptr, 0);
}

void mlg_tiny_config(mlg_config *out) {
    // src/testutil.rs:18-30
    mlg::ModelConfig c;
    c.vocab_size = 4 + 250 + 3;
    c.d_model = 64;
    c.encoder_layers = c.decoder_layers = 2;
    c.encoder_heads = c.decoder_heads = 4;
    c.encoder_ffn = c.decoder_ffn = 128;
    c.max_position_embeddings = 128;
    c.scale_embedding = 1;
    c.bos_token_id = 0;
    c.pad_token_id = 1;
    c.eos_token_id = 2;
    c.decoder_start_token_id = 2;
    c.max_length = 64;
    from_cfg(c, out);
}

int mlg_device_count(int *n) {
    int c = 0;
    const hipError_t e = hipGetDeviceCount(&c);
    if (e != hipSuccess) {
        *n = 0;
        return set_err(MLG_ERR_NO_DEVICE, std::string("no HIP device: ") + hipGetErrorString(e));
    }
    *n = c;
    return MLG_OK;
}

int mlg_ctx_create(int device, mlg_ctx **out) {
    return guarded([&]() -> int {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return set_err(MLG_ERR_NO_DEVICE, "no HIP device");
        if (device < 0 || device >= n) return set_err(MLG_ERR_INVALID, "device ordinal out of range");
        mlg::check_hip(hipSetDevice(device), "hipSetDevice");
        auto c = std::make_unique<mlg_ctx>();
        c->c.device = device;
        mlg::check_hip(hipStreamCreateWithFlags(&c->c.stream, hipStreamNonBlocking), "stream");
        *out = c.release();
        return MLG_OK;
    });
}

void mlg_ctx_destroy(mlg_ctx *ctx) {
    if (!ctx) return;
    if (ctx->c.stream) (void)hipStreamDestroy(ctx->c.stream);
    delete ctx;
}

int mlg_model_load(mlg_ctx *ctx, const char *path, mlg_model **out) {
    return guarded([&]() -> int {
        if (!ctx || !path) return set_err(MLG_ERR_INVALID, "null argument");
        std::lock_guard<std::mutex> lk(ctx->c.mu);
        mlg::check_hip(hipSetDevice(ctx->c.device), "hipSetDevice");
        auto m = std::make_unique<mlg_model>();
        m->m = std::make_unique<mlg::Model>(&ctx->c);
        m->m->load(path);
        *out = m.release();
        return MLG_OK;
    });
}

void mlg_model_free(mlg_model *m) {
    if (!m) return;
    std::lock_guard<std::mutex> lk(m->m->ctx->mu);
    (void)hipSetDevice(m->m->ctx->device);
    delete m;
}

int mlg_model_config(const mlg_model *m, mlg_config *out) {
    if (!m || !out) return set_err(MLG_ERR_INVALID, "null argument");
    from_cfg(m->m->cfg, out);
    return MLG_OK;
}

int64_t mlg_model_weight_bytes(const mlg_model *m) { return m ? int64_t(m->m->weight_bytes) : 0; }

int mlg_model_shortlist_count(const mlg_model *m) { return m ? int(m->m->shortlists.size()) : 0; }

int mlg_model_shortlist_info(const mlg_model *m, int i, const char **code, int *rows) {
    if (!m || i < 0 || i >= int(m->m->shortlists.size())) return set_err(MLG_ERR_INVALID, "no such shortlist");
    const mlg::Shortlist &sl = *m->m->shortlists[size_t(i)];
    if (code) *code = sl.code.c_str();
    if (rows) *rows = int(sl.ids.size());
    return MLG_OK;
}

void mlg_gen_options_default(mlg_gen_options *o) {
    o->beam_size = 1;
    o->max_new_tokens = 0;
    o->length_penalty = 1.f;
    o->sync_every = 4;
    o->max_batch = 32;
    o->fused = 1;
    o->flags = 0;
    o->shortlist = nullptr;
}

}  // extern "C"

namespace {
mlg::GenOptions gen_options(const mlg_gen_options *o) {
    mlg::GenOptions g;
    g.beam_size = o->beam_size;
    g.max_new_tokens = o->max_new_tokens;
    g.length_penalty = o->length_penalty;
    g.sync_every = o->sync_every;
    g.max_batch = o->max_batch;
    g.fused = o->fused != 0 && !(o->flags & MLG_FLAG_NO_GRAPH);
    g.eos_mask = (o->flags & MLG_FLAG_EOS_MASK) != 0;
    if (o->shortlist) g.shortlist = o->shortlist;
    return g;
}
}  // namespace

extern "C" {

int mlg_generate(mlg_model *m, const uint32_t *ids, const uint32_t *lens, int n, uint32_t tgt_lang,
                 const mlg_gen_options *o, uint32_t *out, int out_cap, int *out_len) {
    return guarded([&]() -> int {
        if (!m || n < 0 || (n && (!ids || !lens || !out || !out_len)) || !o) return set_err(MLG_ERR_INVALID, "null argument");
        std::lock_guard<std::mutex> lk(m->m->ctx->mu);
        mlg::check_hip(hipSetDevice(m->m->ctx->device), "hipSetDevice");
        if (tgt_lang >= uint32_t(m->m->cfg.vocab_size)) return set_err(MLG_ERR_INVALID, "target language id out of range");
        const mlg::GenOptions g = gen_options(o);
        if (g.beam_size > 8) return set_err(MLG_ERR_UNSUPPORTED, "beam_size > 8");
        auto src = rows_of(ids, lens, n);
        for (auto &r : src)
            if (r.empty()) return set_err(MLG_ERR_INVALID, "empty source row");
        return write_rows(mlg::generate(*m->m, src, tgt_lang, g), out, out_cap, out_len);
    });
}

int mlg_encode(mlg_model *m, const uint32_t *ids, const uint32_t *lens, int n, mlg_batch **out) {
    return guarded([&]() -> int {
        if (!m || !ids || !lens || n <= 0 || !out) return set_err(MLG_ERR_INVALID, "bad argument");
        std::lock_guard<std::mutex> lk(m->m->ctx->mu);
        mlg::check_hip(hipSetDevice(m->m->ctx->device), "hipSetDevice");
        auto b = std::make_unique<mlg_batch>();
        b->b = m->m->encode(rows_of(ids, lens, n));
        *out = b.release();
        return MLG_OK;
    });
}

void mlg_batch_free(mlg_batch *b) { delete b; }

int mlg_greedy(mlg_model *m, const mlg_batch *b, uint32_t tgt_lang, int max_new, int sync_every, uint32_t flags,
               uint32_t *out, int out_cap, int *out_len) {
    return guarded([&]() -> int {
        if (!m || !b || max_new < 1 || !out || !out_len) return set_err(MLG_ERR_INVALID, "bad argument");
        std::lock_guard<std::mutex> lk(m->m->ctx->mu);
        mlg::check_hip(hipSetDevice(m->m->ctx->device), "hipSetDevice");
        auto rows = m->m->graphs.greedy(*b->b, tgt_lang, max_new, sync_every > 0 ? sync_every : 1,
                                        (flags & MLG_FLAG_EOS_MASK) != 0, !(flags & MLG_FLAG_NO_GRAPH));
        return write_rows(rows, out, out_cap, out_len);
    });
}

int mlg_greedy_top(mlg_model *m, const mlg_batch *b, uint32_t tgt_lang, int max_new, int sync_every, uint32_t flags,
                   uint32_t *out, float *top, int out_cap, int *out_len) {
    return guarded([&]() -> int {
        if (!m || !b || max_new < 1 || !out || !top || !out_len) return set_err(MLG_ERR_INVALID, "bad argument");
        std::lock_guard<std::mutex> lk(m->m->ctx->mu);
        mlg::check_hip(hipSetDevice(m->m->ctx->device), "hipSetDevice");
        std::vector<std::vector<float>> tv;
        auto rows = m->m->graphs.greedy(*b->b, tgt_lang, max_new, sync_every > 0 ? sync_every : 1,
                                        (flags & MLG_FLAG_EOS_MASK) != 0, !(flags & MLG_FLAG_NO_GRAPH), nullptr, &tv);
        const int st = write_rows(rows, out, out_cap, out_len);
        if (st == MLG_OK)
            for (size_t r = 0; r < tv.size(); ++r)
                std::copy(tv[r].begin(), tv[r].end(), top + r * size_t(out_cap));
        return st;
    });
}

int mlg_greedy_sl(mlg_model *m, const mlg_batch *b, uint32_t tgt_lang, const char *code, int max_new, int sync_every,
                  uint32_t flags, uint32_t *out, int out_cap, int *out_len) {
    return guarded([&]() -> int {
        if (!m || !b || !code || max_new < 1 || !out || !out_len) return set_err(MLG_ERR_INVALID, "bad argument");
        const mlg::Shortlist *sl = m->m->shortlist(code);
        if (!sl) return set_err(MLG_ERR_INVALID, std::string("no shortlist for ") + code);
        std::lock_guard<std::mutex> lk(m->m->ctx->mu);
        mlg::check_hip(hipSetDevice(m->m->ctx->device), "hipSetDevice");
        auto rows = m->m->graphs.greedy(*b->b, tgt_lang, max_new, sync_every > 0 ? sync_every : 1,
                                        (flags & MLG_FLAG_EOS_MASK) != 0, !(flags & MLG_FLAG_NO_GRAPH), sl);
        return write_rows(rows, out, out_cap, out_len);
    });
}

int mlg_beam(mlg_model *m, const mlg_batch *b, uint32_t tgt_lang, int max_new, int beam_size, float length_penalty,
             uint32_t flags, uint32_t *out, int out_cap, int *out_len) {
    return guarded([&]() -> int {
        if (!m || !b || max_new < 1 || beam_size < 1 || beam_size > 8 || !out || !out_len)
            return set_err(MLG_ERR_INVALID, "bad argument");
        std::lock_guard<std::mutex> lk(m->m->ctx->mu);
        mlg::check_hip(hipSetDevice(m->m->ctx->device), "hipSetDevice");
        auto rows = m->m->beam(*b->b, tgt_lang, max_new, beam_size, length_penalty, (flags & MLG_FLAG_EOS_MASK) != 0,
                               !(flags & MLG_FLAG_NO_GRAPH));
        return write_rows(rows, out, out_cap, out_len);
    });
}

int mlg_beam_search_host(int b, int k, int max_new, float length_penalty, uint32_t eos, mlg_beam_decode_fn fn,
                         void *user, uint32_t *out, int out_cap, int *out_len) {
    return guarded([&]() -> int {
        if (b < 1 || k < 1 || max_new < 0 || !fn || !out || !out_len) return set_err(MLG_ERR_INVALID, "bad argument");
        const size_t rows = size_t(b) * k;
        std::vector<float> vals(rows * k);
        std::vector<uint32_t> idx(rows * k);
        mlg::BeamMerge merge(b, k, max_new, length_penalty, eos);
        if (fn(user, 1, int(rows), nullptr, nullptr, vals.data(), idx.data()))
            return set_err(MLG_ERR_INVALID, "decode callback failed at step 1");
        for (int step = 1; step <= max_new; ++step) {
            if (merge.merge(step, vals.data(), idx.data())) break;
            if (fn(user, step + 1, int(rows), merge.reorder().data(), merge.next().data(), vals.data(), idx.data()))
                return set_err(MLG_ERR_INVALID, "decode callback failed at step " + std::to_string(step + 1));
        }
        return write_rows(merge.result(), out, out_cap, out_len);
    });
}

int mlg_server_start(mlg_model *m, const mlg_gen_options *defaults, mlg_server **out) {
    return guarded([&]() -> int {
        if (!m || !defaults || !out) return set_err(MLG_ERR_INVALID, "null argument");
        if (defaults->beam_size > 8) return set_err(MLG_ERR_UNSUPPORTED, "beam_size > 8");
        auto s = std::make_unique<mlg_server>();
        s->s = std::make_unique<mlg::Server>(*m->m, gen_options(defaults));
        *out = s.release();
        return MLG_OK;
    });
}

void mlg_server_stop(mlg_server *s) { delete s; }

int mlg_server_submit(mlg_server *s, const uint32_t *ids, const uint32_t *lens, int n, uint32_t src_lang,
                      uint32_t tgt_lang, int beam_size, const char *shortlist, mlg_job **out) {
    return guarded([&]() -> int {
        if (!s || n < 0 || (n && (!ids || !lens)) || !out) return set_err(MLG_ERR_INVALID, "null argument");
        auto j = std::make_unique<mlg_job>();
        j->j = s->s->submit(rows_of(ids, lens, n), src_lang, tgt_lang, beam_size, shortlist ? shortlist : "");
        *out = j.release();
        return MLG_OK;
    });
}

int mlg_job_wait(mlg_job *j, int timeout_ms, int *done) {
    if (!j || !done) return set_err(MLG_ERR_INVALID, "null argument");
    *done = j->j->wait(timeout_ms) ? 1 : 0;
    return MLG_OK;
}

int mlg_job_result(mlg_job *j, uint32_t *out, int out_cap, int *out_len) {
    return guarded([&]() -> int {
        if (!j || (!j->j->src.empty() && (!out || !out_len))) return set_err(MLG_ERR_INVALID, "null argument");
        j->j->wait(-1);
        if (j->j->status != MLG_OK) return set_err(j->j->status, j->j->error);
        return write_rows(j->j->out, out, out_cap, out_len);
    });
}

void mlg_job_free(mlg_job *j) { delete j; }

int mlg_server_stats(const mlg_server *s, int64_t *jobs, int64_t *groups, int64_t *sentences, int64_t *largest_group) {
    if (!s) return set_err(MLG_ERR_INVALID, "null server");
    const mlg::ServerStats st = s->s->stats();
    if (jobs) *jobs = st.jobs;
    if (groups) *groups = st.groups;
    if (sentences) *sentences = st.sentences;
    if (largest_group) *largest_group = st.largest_group;
    return MLG_OK;
}

void mlg_clear_graphs(mlg_model *m) {
    if (!m) return;
    std::lock_guard<std::mutex> lk(m->m->ctx->mu);
    m->m->graphs.clear();
}

int mlg_graph_stats(const mlg_model *m, int *entries, int *graphs, int *capture_enabled) {
    if (!m) return set_err(MLG_ERR_INVALID, "null model");
    *entries = int(m->m->graphs.entries());
    *graphs = int(m->m->graphs.graphs());
    *capture_enabled = m->m->graphs.capture_enabled() ? 1 : 0;
    return MLG_OK;
}

int mlg_graph_cache_keys(const mlg_model *m, int *keys, int cap) {
    if (!m || cap < 0 || (cap && !keys)) return -set_err(MLG_ERR_INVALID, "bad argument");
    std::lock_guard<std::mutex> lk(m->m->ctx->mu);
    const auto k = m->m->graphs.keys();
    for (size_t i = 0; i < k.size() && int(i) < cap; ++i) {
        keys[4 * i] = k[i].b;
        keys[4 * i + 1] = k[i].s;
        keys[4 * i + 2] = k[i].m;
        keys[4 * i + 3] = k[i].graph ? 1 : 0;
    }
    return int(k.size());
}

void mlg_debug_fail_alloc_after(long n) { mlg::set_fail_alloc_after(n); }

int64_t mlg_debug_tile_major(uint32_t type, int N, int K, const void *gguf_rows, void *out, int64_t cap) {
    if (!gguf_rows || N <= 0 || K <= 0 || cap < 0) return -set_err(MLG_ERR_INVALID, "bad argument");
    const size_t tb = mlg::tile_major_bytes(type, N, K);
    if (!tb || !out || cap < int64_t(tb)) return int64_t(tb);
    std::vector<uint8_t> host(mlg::planes_bytes(type, N, K));
    size_t off_s, off_d, total;
    mlg::layout_planes(type, N, K, static_cast<const uint8_t *>(gguf_rows), host.data(), &off_s, &off_d, &total);
    mlg::layout_tile_major(type, N, K, host.data(), off_s, off_d, static_cast<uint8_t *>(out));
    return int64_t(tb);
}

int mlg_bench_stream_read(const void *p, size_t bytes, int mode, int grid, uint32_t *out, void *stream) {
    return hip_status(mlg::stream_read(p, bytes, mode, grid, out, static_cast<hipStream_t>(stream)), "stream_read");
}

int mlg_matrix_upload(mlg_ctx *ctx, uint32_t type, int N, int K, const void *gguf_rows, mlg_matrix **out) {
    return guarded([&]() -> int {
        if (!ctx || !gguf_rows || N <= 0 || K <= 0 || !out) return set_err(MLG_ERR_INVALID, "bad argument");
        mlg::TypeInfo ti;
        if (!mlg::type_info(type, &ti) || type == mlg::GGML_BF16) return set_err(MLG_ERR_UNSUPPORTED, "unsupported type");
        if (K % ti.block_elems) return set_err(MLG_ERR_INVALID, "row length is not a whole number of blocks");
        std::lock_guard<std::mutex> lk(ctx->c.mu);
        mlg::check_hip(hipSetDevice(ctx->c.device), "hipSetDevice");
        std::vector<uint8_t> host(mlg::planes_bytes(type, N, K));
        size_t off_s, off_d, total;
        mlg::layout_planes(type, N, K, static_cast<const uint8_t *>(gguf_rows), host.data(), &off_s, &off_d, &total);
        auto w = std::make_unique<mlg_matrix>();
        w->mem = mlg::dev_alloc(total, "matrix");
        mlg::check_hip(hipMemcpy(w->mem, host.data(), total, hipMemcpyHostToDevice), "upload");
        w->ctx = ctx;
        w->w.type = type;
        w->w.N = N;
        w->w.K = K;
        w->w.q = static_cast<uint8_t *>(w->mem);
        w->w.s = w->w.q + off_s;
        w->w.d = w->w.q + off_d;
        w->w.bytes = total;
        if (const size_t lb = mlg::lane_major_bytes(type, N, K)) {  // as the model's LM heads carry
            std::vector<uint8_t> lm(lb);
            mlg::layout_lane_major(N, K, host.data(), lm.data());
            w->mem_lm = mlg::dev_alloc(lb, "matrix (lane-major quants)");
            w->w.lm = static_cast<uint8_t *>(w->mem_lm);
            mlg::check_hip(hipMemcpy(w->mem_lm, lm.data(), lb, hipMemcpyHostToDevice), "upload");
        }
        if (const size_t tb = mlg::tile_major_bytes(type, N, K)) {  // as the model's q6_K / q4_K ones
            std::vector<uint8_t> tm(tb);
            mlg::layout_tile_major(type, N, K, host.data(), off_s, off_d, tm.data());
            w->mem_tm = mlg::dev_alloc(tb, "matrix (tile-major)");
            w->w.tm = static_cast<uint8_t *>(w->mem_tm);
            mlg::check_hip(hipMemcpy(w->mem_tm, tm.data(), tb, hipMemcpyHostToDevice), "upload");
        }
        *out = w.release();
        return MLG_OK;
    });
}

void mlg_matrix_free(mlg_matrix *w) { delete w; }

int64_t mlg_matrix_bytes(const mlg_matrix *w) { return w ? int64_t(w->w.bytes) : 0; }

int mlg_gemv_max_batch(const mlg_matrix *w) { return w ? mlg::gemv_max_batch(w->w) : 0; }

int mlg_gemv(const mlg_matrix *w, const float *x, int b, float *y, const float *bias, int relu, void *stream) {
    if (!w || !x || !y || b < 1) return set_err(MLG_ERR_INVALID, "bad argument");
    if (b > mlg::gemv_max_batch(w->w)) return set_err(MLG_ERR_INVALID, "batch too large for the GEMV; use mlg_gemm");
    return hip_status(mlg::gemv(w->w, x, w->w.K, b, y, w->w.N, bias, relu != 0, as_stream(stream)), "gemv");
}

int mlg_gemm(const mlg_matrix *w, const float *x, int M, float *y, const float *bias, int relu, void *stream) {
    if (!w || !x || !y || M < 1) return set_err(MLG_ERR_INVALID, "bad argument");
    return guarded([&]() -> int {
        float *ws = w->ctx->c.gemm_workspace();
        return hip_status(mlg::gemm(w->w, x, w->w.K, M, y, w->w.N, bias, relu != 0, nullptr, 0, as_stream(stream), ws,
                                    mlg::kGemmWorkspaceBytes),
                          "gemm");
    });
}

int mlg_gemm_resid(const mlg_matrix *w, const float *x, int M, float *y, const float *bias, int relu, const float *r,
                   void *stream) {
    if (!w || !x || !y || M < 1) return set_err(MLG_ERR_INVALID, "bad argument");
    return guarded([&]() -> int {
        float *ws = w->ctx->c.gemm_workspace();
        return hip_status(mlg::gemm(w->w, x, w->w.K, M, y, w->w.N, bias, relu != 0, r, w->w.N, as_stream(stream), ws,
                                    mlg::kGemmWorkspaceBytes),
                          "gemm");
    });
}

int mlg_gemm_argmax_parts(const mlg_matrix *w, int M) {
    return w && mlg::gemm_argmax_supported(w->w, M) ? mlg::gemm_argmax_parts(w->w, M) : 0;
}

int mlg_gemm_argmax(const mlg_matrix *w, const float *x, int M, int mask_id, float *pv, uint32_t *pi, void *stream) {
    if (!w || !x || !pv || !pi || !mlg::gemm_argmax_supported(w->w, M)) return set_err(MLG_ERR_INVALID, "bad argument");
    int parts = 0;
    return hip_status(mlg::gemm_argmax(w->w, x, w->w.K, M, mask_id, pv, pi, &parts, as_stream(stream)),
                      "gemm_argmax");
}

int mlg_gemv_argmax_parts(const mlg_matrix *w, int b) { return w ? mlg::gemv_argmax_parts(w->w, b) : 0; }

int mlg_gemv_argmax(const mlg_matrix *w, const float *x, int b, int mask_id, float *pv, uint32_t *pi, void *stream) {
    if (!w || !x || !pv || !pi || b < 1 || b > mlg::gemv_max_batch(w->w)) return set_err(MLG_ERR_INVALID, "bad argument");
    int parts = 0;
    return hip_status(mlg::gemv_argmax(w->w, x, w->w.K, b, mask_id, pv, pi, &parts, as_stream(stream)), "gemv_argmax");
}

int mlg_residual_ln(float *x, const float *y, int rows, int d, const float *gamma, const float *beta, float eps,
                    float *ln_out, void *stream) {
    if (!x || !y || !gamma || !beta || !ln_out || rows < 1 || d < 1) return set_err(MLG_ERR_INVALID, "bad argument");
    if (d % 4 || d > 4096 || !aligned16({x, y, gamma, beta, ln_out}))
        return set_err(MLG_ERR_INVALID, "residual_ln: d % 4 == 0, d <= 4096 and 16-byte aligned rows required");
    return hip_status(mlg::residual_ln(x, y, rows, d, gamma, beta, eps, ln_out, as_stream(stream)), "residual_ln");
}

int mlg_layernorm(const float *x, int rows, int d, const float *gamma, const float *beta, float eps, float *out,
                  void *stream) {
    if (!x || !gamma || !beta || !out || rows < 1 || d < 1) return set_err(MLG_ERR_INVALID, "bad argument");
    if (d % 4 || d > 4096 || !aligned16({x, gamma, beta, out}))
        return set_err(MLG_ERR_INVALID, "layernorm: d % 4 == 0, d <= 4096 and 16-byte aligned rows required");
    return hip_status(mlg::layernorm(x, rows, d, gamma, beta, eps, out, as_stream(stream)), "layernorm");
}

int mlg_attn_decode(const float *q, const void *K, const void *V, int b, int H, int hd, int L, const uint32_t *lens,
                    const uint32_t *step, float *out, void *stream) {
    if (!q || !K || !V || !out || b < 1 || H < 1 || L < 1 || (!lens && !step))
        return set_err(MLG_ERR_INVALID, "bad argument");
    if (!mlg::attn_head_size_supported(hd)) return set_err(MLG_ERR_UNSUPPORTED, "head size " + std::to_string(hd));
    return hip_status(mlg::attn_decode(q, static_cast<const __half *>(K), static_cast<const __half *>(V), b, H, hd, L,
                                       lens, lens ? nullptr : step, out, as_stream(stream)),
                      "attn_decode");
}

int mlg_argmax_partial(const float *logits, int b, int V, int mask_id, float *pv, uint32_t *pi, int parts,
                       void *stream) {
    if (!logits || !pv || !pi || b < 1 || V < 1 || parts < 1) return set_err(MLG_ERR_INVALID, "bad argument");
    return hip_status(mlg::argmax_partial(logits, b, V, V, mask_id, pv, pi, parts, as_stream(stream)), "argmax");
}

int mlg_greedy_finalize(const float *pv, const uint32_t *pi, int parts, int b, uint8_t *finished, uint32_t *ids,
                        uint32_t *out, int m, uint32_t *step, uint32_t eos, uint32_t pad, void *stream) {
    if (!pv || !pi || !finished || !ids || !out || !step || b < 1 || parts < 1 || m < 1)
        return set_err(MLG_ERR_INVALID, "bad argument");
    return hip_status(mlg::greedy_finalize(pv, pi, parts, b, finished, ids, out, m, step, eos, pad, as_stream(stream)),
                      "greedy_finalize");
}

size_t mlg_logsoftmax_topk_scratch(int rows, int k) { return mlg::logsoftmax_topk_scratch(rows, k); }

int mlg_logsoftmax_topk(const float *logits, int rows, int V, int k, int mask_id, void *scratch, float *vals,
                        uint32_t *idx, void *stream) {
    if (!logits || !scratch || !vals || !idx || rows < 1 || V < 1 || k < 1 || k > 8)
        return set_err(MLG_ERR_INVALID, "bad argument");
    return hip_status(mlg::logsoftmax_topk(logits, rows, V, k, mask_id, static_cast<float *>(scratch), vals, idx,
                                           as_stream(stream)),
                      "logsoftmax_topk");
}

int mlg_logsoftmax_topk_noalloc(const float *logits, int rows, int V, int k, int mask_id, float *vals, uint32_t *idx,
                                void *stream) {
    if (!logits || !vals || !idx || rows < 1 || V < 1 || k < 1 || k > 8)
        return set_err(MLG_ERR_INVALID, "bad argument");
    if (rows > mlg::kStaticTopkRows)
        return set_err(MLG_ERR_INVALID, "mlg_logsoftmax_topk_noalloc: " + std::to_string(rows) + " rows exceed the " +
                                            std::to_string(mlg::kStaticTopkRows) + "-row static scratch");
    return hip_status(mlg::logsoftmax_topk_static(logits, rows, V, k, mask_id, vals, idx, as_stream(stream)),
                      "logsoftmax_topk_noalloc");
}

int mlg_teacher_forced_logits(mlg_model *m, const uint32_t *ids, const uint32_t *lens, int n, const uint32_t *tgt, int T,
                              int kv_f32, float *logits) {
    return guarded([&]() -> int {
        if (!m || !ids || !lens || n <= 0 || !tgt || T < 1 || !logits) return set_err(MLG_ERR_INVALID, "bad argument");
        std::lock_guard<std::mutex> lk(m->m->ctx->mu);
        mlg::check_hip(hipSetDevice(m->m->ctx->device), "hipSetDevice");
        auto batch = m->m->encode(rows_of(ids, lens, n));
        std::vector<uint32_t> t(tgt, tgt + size_t(n) * T);
        auto out = m->m->teacher_forced(*batch, t, T, kv_f32 != 0);
        std::memcpy(logits, out.data(), out.size() * sizeof(float));
        return MLG_OK;
    });
}

int mlg_bucket(int n, int min, int max) { return mlg::bucket(n, min, max); }

int mlg_budget(const mlg_model *m, int len, int max_new_tokens) {
    return m ? mlg::budget(m->m->cfg, len, max_new_tokens) : 0;
}

int mlg_synchronize(void) { return hip_status(hipDeviceSynchronize(), "synchronize"); }

}  // extern "C"
