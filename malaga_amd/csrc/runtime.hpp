// Decode runtime on one MI355X: weights in HBM, the encoder, the fixed-shape
// decoder state replayed as a hipGraph (src/graph.rs), greedy and beam drivers
// (src/translator.rs), and the translate_batch batching policy.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <list>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "convert.hpp"
#include "kernels.hpp"

namespace mlg {

// Status codes of the C ABI (include/malaga_hip.h).
enum Status : int { OK = 0, ERR_INVALID = 1, ERR_OOM = 2, ERR_HIP = 3, ERR_IO = 4, ERR_FORMAT = 5,
                    ERR_UNSUPPORTED = 6, ERR_NO_DEVICE = 7 };

struct Failure {
    int code;
    std::string msg;
};

// Device allocation with out-of-memory reporting ("OUT_OF_MEMORY" in the message,
// which is what src/graph.rs:215 and src/translator.rs:338-340 match on) and a
// test hook that makes the n-th allocation fail.
void *dev_alloc(size_t bytes, const char *what);
void dev_free(void *p);
void set_fail_alloc_after(long n);  // < 0 disables

// Pinned staging for the small host-to-device uploads of a batch (ids, lengths, flags):
// the copies are asynchronous, and a region of the buffer is rewritten only after the
// event recorded behind every earlier copy out of it has completed.
class Staging {
  public:
    ~Staging();
    // Queues a copy of n bytes from host src to device dst on st (src may be reused at once).
    void upload(void *dst, const void *src, size_t n, hipStream_t st);

  private:
    uint8_t *buf_ = nullptr;
    size_t cap_ = 0, off_ = 0;
    hipEvent_t ev_ = nullptr;
    bool pending_ = false;
};

struct Context {
    int device = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;  // one caller at a time per context (src/graph.rs:152-155)
    float *gemm_ws = nullptr;  // split-K workspace of the MFMA GEMM (kGemmWorkspaceBytes)
    Staging staging;           // uploads on `stream`
    // Allocates the workspace on first use (never inside a graph capture: the first
    // eager step or the encoder reaches it first).
    float *gemm_workspace();
    ~Context();
};

struct Linear {
    DevMatrix w;
    float *b = nullptr;
};
struct LNorm {
    float *g = nullptr, *b = nullptr;
};
struct EncLayer {
    LNorm attn_norm, ffn_norm;
    Linear qkv, out, up, down;
};
struct DecLayer {
    LNorm attn_norm, cross_norm, ffn_norm;
    Linear qkv, out, cross_q, cross_out, up, down;  // cross_attn_kv: Model::cross_kv
};

// Reduced LM head of one target language (src/model.rs:229-250): rows of token_embd
// for the sorted vocabulary ids `ids`, stored as lm_head.{code}.weight.
struct Shortlist {
    std::string code;
    DevMatrix head;
    std::vector<uint32_t> ids;  // sorted
    uint32_t *d_ids = nullptr;  // same ids on the device
    // Row of `head` holding vocabulary id `id`, or -1.
    int row(uint32_t id) const {
        auto it = std::lower_bound(ids.begin(), ids.end(), id);
        return it != ids.end() && *it == id ? int(it - ids.begin()) : -1;
    }
    bool contains(uint32_t id) const { return row(id) >= 0; }
};

// Encoded sources: per decoder layer cross K/V [b][H][s][hd] in f32, as
// Nllb::encode_cross returns them (src/model.rs:463-477); a decode state keeps them in f16
// (the graph step, src/graph.rs:94-97) or f32 (the generic path).
struct Batch {
    int b = 0, s = 0;
    std::vector<uint32_t> lens;
    std::vector<uint32_t> ids;    // [b][s] source ids, right-padded with pad
    std::vector<float *> ck, cv;  // per decoder layer, inside `block`
    void *block = nullptr;        // one allocation for every layer's cross K/V
    ~Batch();
};

// src/graph.rs:23-49
struct StaticState {
    int b = 0, s = 0, m = 0;
    uint32_t *ids = nullptr, *step = nullptr, *lens = nullptr, *out = nullptr;
    float *outv = nullptr;  // [b][m]: the winning logit of each greedy token (parity hook)
    uint32_t *err = nullptr;  // set by the greedy finalize when a live row has no finite logit
    uint8_t *finished = nullptr;
    // self and cross K/V per layer: f16 (kc ..; the fused graph step, kernels/malaga.cu:
    // 142-154) or, with kv32, f32 (kc32 ..; the generic decode path's candle KvCache and
    // cross K/V, src/model.rs:195-227, 504-540)
    bool kv32 = false;
    std::vector<__half *> kc, vc, ck, cv;
    std::vector<float *> kc32, vc32, ck32, cv32;
    // workspace (nothing is allocated inside a step)
    float *x = nullptr, *h = nullptr, *y = nullptr, *att = nullptr, *q = nullptr, *qkv = nullptr, *u = nullptr;
    float *xb = nullptr, *qc = nullptr;  // second residual buffer and cross queries (fused step)
    float *part = nullptr;                // attention partial sums [parts][b][d] (fused step)
    float *part2 = nullptr;               // second partials buffer: the cross launch reads part, writes part2
    uint32_t *rows = nullptr;             // beam: [b][m] cache row holding slot j of row r (null: r)
    uint32_t *row_src = nullptr;          // [b] source row of each state row (reset_state)
    // shortlist decoding (src/graph.rs:40-48): candidates are the shortlist rows and the
    // source tokens; the next input embedding is shortlist row sl_row[r] or, where
    // src_row[r] != kNoRow, source position src_row[r] of src_emb.
    const Shortlist *sl = nullptr;
    uint32_t *src_ids = nullptr;          // [b][s] pad beyond each row's length
    float *src_emb = nullptr;             // [b][s][d] token_embd rows of src_ids
    uint32_t *sl_row = nullptr, *src_row = nullptr;
    float *spv = nullptr;                 // [b][s] source-token logits
    uint32_t *spi = nullptr;              // [b][s] their candidate indices
    uint8_t *src_q = nullptr;             // lazy embeddings: token_embd rows of src_ids (device layout)
    uint32_t *src_iota = nullptr;         // lazy embeddings: 0 .. b*s-1
    bool fused = false;                   // decoder step uses the fused kernels of k_step.hip
    float *logits = nullptr, *pv = nullptr;
    uint32_t *pi = nullptr;
    int parts = 0;
    // decode-GEMM step (batches of 5..64 rows): [b][d / 16][2] f64 sums of the residual
    // stream and its squares per 16 columns, written with x by every projection that adds
    // to it and read by the next LayerNorm (null: the split-K step)
    double *lnstat = nullptr;
    size_t bytes = 0;
    std::vector<void *> owned;
    ~StaticState();
};

class Model;

// src/graph.rs:149-335: bucketed static states + captured step graphs, LRU by bytes.
class GraphCache {
  public:
    explicit GraphCache(Model *m);
    ~GraphCache();
    bool capture_enabled() const { return capture_; }
    void clear();
    // Greedy decoding of an encoded batch; rows stripped at EOS (src/graph.rs:204-298).
    // sl: decode over the shortlist + source tokens (src/graph.rs:204-298 with a shortlist).
    // top (optional): receives each row's winning logits, one per returned token.
    std::vector<std::vector<uint32_t>> greedy(const Batch &src, uint32_t tgt_lang, int max_new, int sync_every,
                                              bool eos_mask, bool use_graph, const Shortlist *sl = nullptr,
                                              std::vector<std::vector<float>> *top = nullptr);
    size_t entries() const { return entries_.size(); }
    size_t graphs() const;
    // Bucket keys (b, s, m) of the cached states, least recently used first, and
    // whether each holds a captured graph.
    struct Key {
        int b, s, m;
        bool graph;
    };
    std::vector<Key> keys() const;

  private:
    struct Entry {
        int b, s, m;
        const Shortlist *sl = nullptr;  // part of the key (src/graph.rs:157)
        std::unique_ptr<StaticState> st;
        hipGraphExec_t exec = nullptr;
        uint64_t last_used = 0;
        size_t bytes() const;
    };
    std::vector<std::vector<uint32_t>> run(const Batch &src, uint32_t tgt_lang, int max_new, int sync_every,
                                           bool eos_mask, bool use_graph, const Shortlist *sl,
                                           std::vector<std::vector<float>> *top);
    void evict(const Entry *keep);
    static void trim_graph_memory();
    Model *model_;
    std::list<Entry> entries_;
    uint64_t clock_ = 0;
    size_t max_bytes_;
    bool capture_;
    uint8_t *fin_host_ = nullptr;  // pinned copy of the finished flags
    size_t fin_cap_ = 0;
    hipEvent_t fin_ev_ = nullptr;
};

class Model {
  public:
    Model(Context *ctx) : ctx(ctx), graphs(this) {}
    ~Model();
    void load(const std::string &path);  // throws Failure

    Context *ctx;
    ModelConfig cfg;
    DevMatrix embed;  // token_embd, also the tied LM head (q == nullptr: still on the host, see ensure_embed)
    float *pos = nullptr;
    int n_pos = 0;
    float embed_scale = 1.f;
    std::vector<EncLayer> enc;
    std::vector<DecLayer> dec;
    LNorm enc_norm, dec_norm;
    // every decoder layer's cross_attn_kv [2d, d] stacked layer after layer into one
    // [L * 2d, d] matrix (and bias), so that the encoder computes all cross K/V at once
    Linear cross_kv;
    std::vector<std::unique_ptr<Shortlist>> shortlists;  // src/model.rs:403-412
    size_t weight_bytes = 0;
    GraphCache graphs;

    // src/model.rs:463-500 (encoder + cross K/V of every decoder layer)
    std::unique_ptr<Batch> encode(const std::vector<std::vector<uint32_t>> &src);
    // Shortlist of a target-language code, or null (src/model.rs:439-442).
    const Shortlist *shortlist(const std::string &code) const;
    // Embedding::on_device (src/model.rs:275-305): with MALAGA_LAZY_EMBEDDINGS set and a
    // shortlist in the file, token_embd stays on the host until exact decoding needs the
    // full LM head; this uploads it (once).  Never called inside a graph capture.
    void ensure_embed();
    bool embed_resident() const { return embed.q != nullptr; }
    // logits: keep a [b][V] logits buffer; row_map: beam-search cache-row map (rows);
    // sl: buffers of shortlist decoding (greedy only).
    // kv32: f32 K/V caches (the generic path; never the fused step kernels)
    std::unique_ptr<StaticState> new_state(int b, int s, int m, bool logits, bool row_map = false,
                                           const Shortlist *sl = nullptr, bool kv32 = false);
    // src/model.rs:552-612: one decoder step on fixed buffers.  greedy: argmax +
    // bookkeeping, else logits into st.logits and ++step.
    void step(StaticState &st, bool greedy, int mask_id);
    // Whether the fused step kernels cover a state of b rows with caches of m / s slots.
    bool fusable(int b, int m, int s) const;
    void reset_state(StaticState &st, const Batch &src, const std::vector<uint32_t> &row_of, uint32_t start);
    // Shortlist state: every row's next input embedding is the shortlist row of `id`.
    void set_shortlist_input(StaticState &st, uint32_t id);
    // src/translator.rs:250-335.  use_graph: replay one captured step + top-k per
    // beam step (off when capture is disabled for the cache).
    // Decodes on f32 K/V like the reference's Nllb::encode/decode path.
    std::vector<std::vector<uint32_t>> beam(const Batch &src, uint32_t tgt_lang, int max_new, int k, float lp,
                                            bool eos_mask, bool use_graph = true);
    // src/translator.rs:195-199, 214-241: greedy decoding on the generic path (GenOptions::
    // fused = false): f32 K/V, every step launched eagerly, the finished flags read every
    // sync_every steps.
    std::vector<std::vector<uint32_t>> greedy_generic(const Batch &src, uint32_t tgt_lang, int max_new,
                                                      int sync_every, bool eos_mask);
    // Logits after feeding tgt[:, t] at position t, for t < T: [b][T][V] (parity tests);
    // kv32: on f32 K/V (the generic path), else f16 (the graph step).
    std::vector<float> teacher_forced(const Batch &src, const std::vector<uint32_t> &tgt, int T, bool kv32 = false);

  private:
    std::vector<void *> owned_;
    std::vector<uint8_t> embed_host_;  // token_embd GGUF rows while not resident
    // token_embd rows of host ids as an n-row device matrix in buf (planes_bytes(type, n, d))
    DevMatrix gather_embed(const uint32_t *ids, int n, uint8_t *buf);
    // Encoder scratch (ids, activations): grow-only, reused by every encode call, so a
    // call allocates only the cross K/V it returns.
    void *enc_ws_ = nullptr;
    size_t enc_ws_bytes_ = 0;
    Linear load_linear(class GgufFile &g, const std::string &name, int n, int k);
    LNorm load_ln(class GgufFile &g, const std::string &name, int d);
    float *upload_f32(class GgufFile &g, const std::string &name, int64_t n);
    // q6_K / q4_K: also the tile-major copy (DevMatrix::tm); head: the lane-major quant copy of a
    // q6_K LM head (DevMatrix::lm)
    DevMatrix upload_matrix(class GgufFile &g, const std::string &name, int n, int k, bool head = false);
    void upload_lane_major(DevMatrix &m, const uint8_t *q_plane);
    void upload_tile_major(DevMatrix &m, const uint8_t *planes, size_t off_s, size_t off_d);
    Linear load_stacked(class GgufFile &g, const std::string &suffix, int layers, int n, int k);
    void matmul(const Linear &l, const float *x, int rows, float *y, bool relu, const float *resid);
    // final_ln: end with h = dec_norm(x + y); otherwise return x for the LM head to
    // fold that LayerNorm into its launch (the residual buffer holding x)
    float *step_fused(StaticState &st, bool final_ln = true);
    // ln_x: x of the final LayerNorm when the head computes it (step_fused(st, false))
    void lm_head(StaticState &st, bool greedy_mode, int mask_id, const float *ln_x = nullptr);
    // batches of 5..64 rows: eight launches per layer (decode GEMMs with the LayerNorms
    // folded in, k_dgemm.hip); false when a matrix or the batch does not fit them
    bool dgemm_step_ok(int b) const;
    void step_dgemm(StaticState &st, bool greedy_mode, int mask_id);
    bool split_k_step_ = false;  // MALAGA_SPLIT_K_STEP=1: batches > 4 keep the split-K GEMMs
    bool no_fuse_ = false;  // MALAGA_NO_FUSED_STEP=1 forces the unfused step
    bool split_cross_ = false;  // MALAGA_SPLIT_CROSS_STEP=1: cross_q and cross attention as two launches
};

void check_hip(hipError_t e, const char *what);  // throws Failure

struct GenOptions {
    int beam_size = 1;
    int max_new_tokens = 0;  // 0 = 2*len + 16
    float length_penalty = 1.f;
    int sync_every = 4;
    int max_batch = 32;
    bool fused = true;
    bool eos_mask = false;  // benchmark-only: fixed output lengths
    std::string shortlist;  // target-language code whose shortlist greedy decoding uses ("" = off)
};

// src/translator.rs:136-207 on token ids: sort by length, batch, per-row budget,
// OOM batch halving.  Output order matches input order.
std::vector<std::vector<uint32_t>> generate(Model &m, const std::vector<std::vector<uint32_t>> &src, uint32_t tgt_lang,
                                            const GenOptions &o);
// One batch (src/translator.rs:175-207).
std::vector<std::vector<uint32_t>> generate_to(Model &m, const std::vector<std::vector<uint32_t>> &src,
                                               uint32_t tgt_lang, const GenOptions &o);
int budget(const ModelConfig &c, int len, int max_new_tokens);
// src/graph.rs:138-140
int bucket(int n, int min, int max);

}  // namespace mlg
