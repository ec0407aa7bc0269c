/*
 * malaga_hip.h -- C ABI of libmalaga_hip.so, the MI355X (gfx950) backend for
 * malaga's NLLB/M2M100 GGUF decode path.
 *
 * Plain C types only (no torch, no HIP types): a Rust FFI crate, ctypes or any
 * C caller binds it directly.  Each entry point cites the reference interface it
 * replaces (paths relative to rzafiamy/malaga, crates/malaga-core/).
 *
 * Conventions
 *   - Every int-returning function returns MLG_OK (0) or an MLG_ERR_* status;
 *     mlg_last_error() then holds a thread-local message.  Out-of-memory
 *     messages contain "OUT_OF_MEMORY", the substring the reference's retry
 *     logic matches (src/graph.rs:215, src/translator.rs:338-340).
 *   - Host buffers are caller-owned; the library copies in and out.  All device
 *     memory of contexts, models, batches and graph states is library-owned.
 *   - A context (and the models loaded on it) is used by one thread at a time;
 *     calls take the context's mutex (src/graph.rs:152-155).
 *   - Kernel-level entry points take device pointers and a hipStream_t passed
 *     as void* (NULL = the context-independent default stream).
 */
#ifndef MALAGA_HIP_H
#define MALAGA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    MLG_OK = 0,
    MLG_ERR_INVALID = 1,
    MLG_ERR_OOM = 2,
    MLG_ERR_HIP = 3,
    MLG_ERR_IO = 4,
    MLG_ERR_FORMAT = 5,
    MLG_ERR_UNSUPPORTED = 6,
    MLG_ERR_NO_DEVICE = 7
};

/* ggml type ids (GGUF spec) accepted by the codecs and kernels */
enum { MLG_F32 = 0, MLG_F16 = 1, MLG_Q8_0 = 8, MLG_Q4_K = 12, MLG_Q5_K = 13, MLG_Q6_K = 14, MLG_BF16 = 30 };

/* src/convert.rs:25-91 presets (Preset and its linear / ffn_down / embedding types) */
enum { MLG_PRESET_F32 = 0, MLG_PRESET_F16, MLG_PRESET_Q8_0, MLG_PRESET_Q6K, MLG_PRESET_Q5KM, MLG_PRESET_Q4KM };

/* synthetic checkpoints (tests / benchmarks) */
enum { MLG_INIT_TESTUTIL = 0, MLG_INIT_NORMAL = 1, MLG_INIT_NORMAL_RICH = 2 };

/* generation flags */
enum {
    MLG_FLAG_EOS_MASK = 1, /* benchmark-only: EOS logit = -inf, fixed output lengths (no reference counterpart) */
    MLG_FLAG_NO_GRAPH = 2  /* run the static step eagerly (MALAGA_NO_HIP_GRAPH for one call) */
};

typedef struct mlg_ctx mlg_ctx;
typedef struct mlg_model mlg_model;
typedef struct mlg_batch mlg_batch;
typedef struct mlg_matrix mlg_matrix;

/* Hyper-parameters: src/config.rs:14-39 (field for field). */
typedef struct {
    int vocab_size, d_model, encoder_layers, decoder_layers, encoder_heads, decoder_heads;
    int encoder_ffn, decoder_ffn, max_position_embeddings, max_length, scale_embedding;
    int bos_token_id, pad_token_id, eos_token_id, decoder_start_token_id;
} mlg_config;

/* src/translator.rs:15-53 GenOptions. */
typedef struct {
    int beam_size;        /* 1 = greedy */
    int max_new_tokens;   /* 0 = None: 2 * src_len + 16, capped by max_length */
    float length_penalty;
    int sync_every;
    int max_batch;
    int fused;            /* GenOptions::fused (src/translator.rs:184-201).  1: greedy runs the graph
                             cache's static step (f16 K/V, replayed as a hipGraph).  0: greedy runs the
                             generic decoder (Nllb::decode semantics: f32 K/V caches and cross K/V,
                             eager launches).  Beam search always runs the generic decoder (f32 K/V);
                             fused = 1 replays its captured step, 0 launches it eagerly. */
    uint32_t flags;       /* MLG_FLAG_* */
    const char *shortlist; /* GenOptions::shortlist (--fast-vocab): the target-language code whose
                              shortlist greedy decoding uses when the model has one that holds
                              decoder_start and tgt_lang (src/translator.rs:184-194); NULL = exact */
} mlg_gen_options;

const char *mlg_last_error(void);
const char *mlg_version(void);

/* ---- block codecs (candle-core 0.11 QTensor quantize/dequantize, src/convert.rs:128-136) ---- */
int mlg_type_info(uint32_t type, int *block_elems, int *block_bytes);
int64_t mlg_type_bytes(uint32_t type, int64_t n);
int mlg_quantize(uint32_t type, const float *x, int64_t n, void *out);
int mlg_dequantize(uint32_t type, const void *in, int64_t n, float *out);

/* ---- conversion (src/convert.rs:196-318) ---- */
int mlg_preset_from_name(const char *name, int *preset);
/* Supplies the f32 data of a Hugging Face tensor; return 0 on success. */
typedef int (*mlg_tensor_fn)(void *user, const char *hf_name, int64_t numel, float *out);
int mlg_convert(const char *out_path, const mlg_config *cfg, int preset, const char *model_name,
                const char *tokenizer_json, mlg_tensor_fn fn, void *user);
/* Synthetic checkpoint converted like mlg_convert (MLG_INIT_TESTUTIL restates src/testutil.rs:16-101). */
int mlg_write_synthetic(const char *out_path, const mlg_config *cfg, int preset, int init, uint64_t seed,
                        float std_dev, const char *model_name);
/* Per-language shortlist (reduced LM head, src/convert.rs:176-233): the writer adds ids 0..3
   and lang_id, sorts, and stores token_embd's rows for the ids as lm_head.{code}.weight and
   the ids as nllb.shortlist.{code}.  The reference tokenizes a corpus for `ids`; here the
   caller supplies them. */
typedef struct {
    const char *code;     /* language code, e.g. "fra_Latn" */
    uint32_t lang_id;     /* the language token (kept: it is fed to the decoder) */
    const uint32_t *ids;  /* vocabulary ids of the shortlist (any order, duplicates allowed) */
    int n_ids;
} mlg_shortlist_spec;
/* mlg_convert / mlg_write_synthetic plus shortlists (src/convert.rs:218-233, 303). */
int mlg_convert_sl(const char *out_path, const mlg_config *cfg, int preset, const char *model_name,
                   const char *tokenizer_json, mlg_tensor_fn fn, void *user, const mlg_shortlist_spec *sl, int n_sl);
int mlg_write_synthetic_sl(const char *out_path, const mlg_config *cfg, int preset, int init, uint64_t seed,
                           float std_dev, const char *model_name, const mlg_shortlist_spec *sl, int n_sl);
/* The tiny test model of src/testutil.rs:18-30. */
void mlg_tiny_config(mlg_config *out);

/* ---- device context and model (src/translator.rs:62-73, src/model.rs:343-433) ---- */
int mlg_device_count(int *n);
int mlg_ctx_create(int device, mlg_ctx **out);
void mlg_ctx_destroy(mlg_ctx *ctx);
int mlg_model_load(mlg_ctx *ctx, const char *gguf_path, mlg_model **out);
void mlg_model_free(mlg_model *m);
int mlg_model_config(const mlg_model *m, mlg_config *out);
int64_t mlg_model_weight_bytes(const mlg_model *m);
/* Nllb::shortlist_langs / shortlist (src/model.rs:439-447): number of shortlists, and the
   language code and row count of shortlist i (code valid while the model lives). */
int mlg_model_shortlist_count(const mlg_model *m);
int mlg_model_shortlist_info(const mlg_model *m, int i, const char **code, int *rows);

/* ---- translation on token ids ---- */
void mlg_gen_options_default(mlg_gen_options *o);
/* Translator::translate_batch (src/translator.rs:136-167) + generate_to (175-207) on
 * already-tokenized sources: n rows, row i = ids[off_i .. off_i + lens[i]).  out is
 * [n][out_cap]; out_len[i] receives the length of row i (without specials). */
int mlg_generate(mlg_model *m, const uint32_t *ids, const uint32_t *lens, int n, uint32_t tgt_lang,
                 const mlg_gen_options *o, uint32_t *out, int out_cap, int *out_len);

/* GraphCache boundary (src/graph.rs:182-223): encode once, then decode. */
/* Nllb::encode_cross (src/model.rs:463-477). */
int mlg_encode(mlg_model *m, const uint32_t *ids, const uint32_t *lens, int n, mlg_batch **out);
void mlg_batch_free(mlg_batch *b);
/* GraphCache::greedy (src/graph.rs:204-223); rows stripped at EOS. */
int mlg_greedy(mlg_model *m, const mlg_batch *b, uint32_t tgt_lang, int max_new, int sync_every, uint32_t flags,
               uint32_t *out, int out_cap, int *out_len);
/* mlg_greedy, plus top [n][out_cap]: the logit of each returned token as the step's
   argmax saw it (the LM head's winning value, before the finished / pad rule).  Parity
   hook for tests of the fused argmax head; no counterpart in the reference. */
int mlg_greedy_top(mlg_model *m, const mlg_batch *b, uint32_t tgt_lang, int max_new, int sync_every, uint32_t flags,
                   uint32_t *out, float *top, int out_cap, int *out_len);
/* GraphCache::greedy with Some(shortlist) (src/graph.rs:204-298, src/model.rs:597-606): the
   candidates of each step are the shortlist rows of language `code` and the batch's source
   tokens.  MLG_ERR_INVALID if the model has no such shortlist or it lacks decoder_start or
   tgt_lang ("token missing from the shortlist", src/graph.rs:125). */
int mlg_greedy_sl(mlg_model *m, const mlg_batch *b, uint32_t tgt_lang, const char *code, int max_new, int sync_every,
                  uint32_t flags, uint32_t *out, int out_cap, int *out_len);
/* Translator::beam_search (src/translator.rs:250-335) on the generic decoder's f32 K/V caches
   (src/model.rs:195-227).  One decoder step + top-k is captured once and replayed per step
   (MLG_FLAG_NO_GRAPH: eager); MLG_FLAG_EOS_MASK as for mlg_greedy. */
int mlg_beam(mlg_model *m, const mlg_batch *b, uint32_t tgt_lang, int max_new, int beam_size, float length_penalty,
             uint32_t flags, uint32_t *out, int out_cap, int *out_len);
/* The host half of Translator::beam_search (src/translator.rs:250-335: candidate merge,
   length penalty, early stop, padding, final pick) over a caller's decoder: for callers
   that run the decoder step and top-k themselves, and for tests of the merge rules.
   decode(user, step, rows, reorder, next, vals, idx) is called for step 1 with
   reorder = next = NULL (the rows have just decoded [decoder_start, tgt_lang]); for
   step s > 1 row r first continues row reorder[r] (st.reorder, translator.rs:323) and
   is fed next[r] (translator.rs:324-325).  It writes the top-k log-probs and tokens of
   every row, best first with ties to the lowest token (translator.rs:343-358), into
   vals/idx [rows][k] (rows = b * k) and returns 0, or nonzero to stop with
   MLG_ERR_INVALID.  No device is used.  out is [b][out_cap] as mlg_generate. */
typedef int (*mlg_beam_decode_fn)(void *user, int step, int rows, const uint32_t *reorder, const uint32_t *next,
                                  float *vals, uint32_t *idx);
int mlg_beam_search_host(int b, int k, int max_new, float length_penalty, uint32_t eos, mlg_beam_decode_fn fn,
                         void *user, uint32_t *out, int out_cap, int *out_len);

/* ---- dynamic batching caller (crates/malaga/src/server.rs:74-112) ----
   One inference thread per server owns the model.  Jobs submitted from any thread are
   queued; the thread takes every queued job, groups those with the same (src_lang,
   tgt_lang, beam_size, shortlist) in order of first arrival (server.rs:83-90) and decodes
   each group as one mlg_generate call with the server's options (server.rs:93-112), so
   requests that arrive while the GPU is busy share the next batch.  The model must
   outlive the server; other calls on the same model wait for the running group. */
typedef struct mlg_server mlg_server;
typedef struct mlg_job mlg_job;
int mlg_server_start(mlg_model *m, const mlg_gen_options *defaults, mlg_server **out);
/* Finishes every queued job, then stops the thread. */
void mlg_server_stop(mlg_server *s);
/* n sentences (as mlg_generate); beam_size <= 0 = the server's, clamped to 1..8
   (server.rs:64); shortlist: language code or NULL (GenOptions::shortlist).  Bad ids,
   empty rows or a stopped server: MLG_ERR_INVALID at submission. */
int mlg_server_submit(mlg_server *s, const uint32_t *ids, const uint32_t *lens, int n, uint32_t src_lang,
                      uint32_t tgt_lang, int beam_size, const char *shortlist, mlg_job **out);
/* *done = 1 once the job has its result; timeout_ms < 0 waits without limit. */
int mlg_job_wait(mlg_job *j, int timeout_ms, int *done);
/* Waits for the job, then returns its status (the group's error, if any, with its
   message in mlg_last_error) and its rows as mlg_generate does. */
int mlg_job_result(mlg_job *j, uint32_t *out, int out_cap, int *out_len);
void mlg_job_free(mlg_job *j);
/* Jobs and sentences decoded, groups run, largest group in sentences. */
int mlg_server_stats(const mlg_server *s, int64_t *jobs, int64_t *groups, int64_t *sentences, int64_t *largest_group);

/* GraphCache::clear (src/graph.rs:192-200). */
void mlg_clear_graphs(mlg_model *m);
int mlg_graph_stats(const mlg_model *m, int *entries, int *graphs, int *capture_enabled);
/* The cache's entries, least recently used first (the eviction order of src/graph.rs:301-323):
   up to cap rows of (batch bucket, source bucket, output bucket, has a graph) into keys
   [cap][4]; returns the number of entries (or a negative status).  Introspection for
   tests; no counterpart in the reference. */
int mlg_graph_cache_keys(const mlg_model *m, int *keys, int cap);
/* Test hook: the n-th following device allocation fails with MLG_ERR_OOM (n < 0: off). */
void mlg_debug_fail_alloc_after(long n);
/* Test hook: the tile-major copy the MFMA GEMMs read for q6_K / q4_K GGUF rows [N][K] (K % 256
   == 0; rows past N padded to a multiple of 16 with zeros): returns its size in bytes
   (0: the type or shape has none) and
   writes it to out when cap holds it.  No counterpart in the reference (the layout is this
   backend's). */
int64_t mlg_debug_tile_major(uint32_t type, int N, int K, const void *gguf_rows, void *out, int64_t cap);
/* Streaming-read ceiling, the reference point of the LM head's roofline (measurement only;
   no counterpart in the reference): `grid` workgroups of 256 threads read every 16-byte word
   of p[0, bytes) once, 8 loads of 16 bytes in flight per thread; mode 0 ordinary loads,
   1 non-temporal loads, 2 direct-to-LDS loads (global_load_lds_dwordx4).  bytes % 16 == 0,
   p 16-byte aligned; out: 4 bytes the kernel may write (so that the loads are kept). */
int mlg_bench_stream_read(const void *p, size_t bytes, int mode, int grid, uint32_t *out, void *stream);

/* ---- kernel-level entry points (microbenchmarks and tests; device pointers) ---- */
/* A GGUF matrix [N][K] of `type` (raw GGUF row bytes from the host) uploaded in the device layout. */
int mlg_matrix_upload(mlg_ctx *ctx, uint32_t type, int N, int K, const void *gguf_rows, mlg_matrix **out);
void mlg_matrix_free(mlg_matrix *w);
int64_t mlg_matrix_bytes(const mlg_matrix *w);
/* QMatMul::forward (src/model.rs:571-607): y[b][N] = x[b][K] W^T (+ bias) (relu). */
int mlg_gemv(const mlg_matrix *w, const float *x, int b, float *y, const float *bias, int relu, void *stream);
int mlg_gemv_max_batch(const mlg_matrix *w);
int mlg_gemm(const mlg_matrix *w, const float *x, int M, float *y, const float *bias, int relu, void *stream);
/* As mlg_gemm, plus a residual: y = x W^T + bias + r (r may be y itself), then relu.
 * The residual adds of EncoderLayer::forward (src/model.rs:150-153) folded into the
 * projections that precede them. */
int mlg_gemm_resid(const mlg_matrix *w, const float *x, int M, float *y, const float *bias, int relu, const float *r,
                   void *stream);
/* The same for decode batches of up to 64 rows on the MFMA units (X resident in LDS up
 * to 32 rows, staged per K step above): partials [M][mlg_gemm_argmax_parts(w, M)];
 * mlg_gemm_argmax_parts returns 0 where this form does not apply. */
int mlg_gemm_argmax_parts(const mlg_matrix *w, int M);
int mlg_gemm_argmax(const mlg_matrix *w, const float *x, int M, int mask_id, float *pv, uint32_t *pi, void *stream);
/* LM head + first argmax pass (kernels/malaga.cu:247-280 fused into the GEMV):
 * partials pv/pi [b][mlg_gemv_argmax_parts(w, b)] (one per workgroup launched). */
int mlg_gemv_argmax_parts(const mlg_matrix *w, int b);
int mlg_gemv_argmax(const mlg_matrix *w, const float *x, int b, int mask_id, float *pv, uint32_t *pi, void *stream);
/* bias_residual_ln (kernels/malaga.cu:89-105 semantics) with the bias already in y: x += y,
   ln_out = LayerNorm(x) (biased variance); d % 4 == 0, d <= 4096. */
int mlg_residual_ln(float *x, const float *y, int rows, int d, const float *gamma, const float *beta, float eps,
                    float *ln_out, void *stream);
int mlg_layernorm(const float *x, int rows, int d, const float *gamma, const float *beta, float eps, float *out,
                  void *stream);
/* attn_decode (kernels/malaga.cu:165-227 semantics). K, V: f16 [b][H][L][hd]; hd one of 8, 16,
   32, 64, 128, 256 (else MLG_ERR_UNSUPPORTED); n = lens[row] keys, or *step + 1 without lens. */
int mlg_attn_decode(const float *q, const void *K, const void *V, int b, int H, int hd, int L, const uint32_t *lens,
                    const uint32_t *step, float *out, void *stream);
/* argmax_partial (kernels/malaga.cu:247-280): pv/pi [b][parts]. */
int mlg_argmax_partial(const float *logits, int b, int V, int mask_id, float *pv, uint32_t *pi, int parts,
                       void *stream);
/* greedy_finalize (kernels/malaga.cu:290-326). */
int mlg_greedy_finalize(const float *pv, const uint32_t *pi, int parts, int b, uint8_t *finished, uint32_t *ids,
                        uint32_t *out, int m, uint32_t *step, uint32_t eos, uint32_t pad, void *stream);
/* log_softmax + topk (src/translator.rs:272, 343-358); scratch of mlg_logsoftmax_topk_scratch bytes. */
size_t mlg_logsoftmax_topk_scratch(int rows, int k);
int mlg_logsoftmax_topk(const float *logits, int rows, int V, int k, int mask_id, void *scratch, float *vals,
                        uint32_t *idx, void *stream);
/* mlg_logsoftmax_topk with no workspace argument and no allocation of any kind, for callers
   that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
   forbid hipMalloc).  No counterpart in the reference.  The partial results live in a static
   device array of the library (1.125 MiB, held by each GPU it runs on until the process ends),
   so rows <= 256 (more: MLG_ERR_INVALID before anything runs).  Call with the stream's device
   current.  Calls on one GPU share the array: calls that overlap on one GPU race. */
int mlg_logsoftmax_topk_noalloc(const float *logits, int rows, int V, int k, int mask_id, float *vals, uint32_t *idx,
                                void *stream);
/* Logits after feeding tgt[i][t] at decoder position t (t < T), eagerly: out is [n][T][vocab].
 * kv_f32 = 0: K/V caches in f16, as the graph step stores them (kernels/malaga.cu:142-154);
 * kv_f32 = 1: in f32, as Nllb::decode keeps them (src/model.rs:195-227, 514-540).
 * Parity hook; no counterpart in the reference. */
int mlg_teacher_forced_logits(mlg_model *m, const uint32_t *ids, const uint32_t *lens, int n, const uint32_t *tgt, int T,
                              int kv_f32, float *logits);
/* src/graph.rs:138-140 */
int mlg_bucket(int n, int min, int max);
/* per-sentence output budget, src/translator.rs:181-182 */
int mlg_budget(const mlg_model *m, int len, int max_new_tokens);
int mlg_synchronize(void);

#ifdef __cplusplus
}
#endif
#endif
