/* oracle.h -- CPU restatement of malaga's dequantized NLLB decode path.
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline); never linked into
 * the product library. */
#ifndef MALAGA_ORACLE_H
#define MALAGA_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_KV_F16 = 1, ORC_EOS_MASK = 2 };

typedef struct {
    int vocab_size, d_model, encoder_layers, decoder_layers, encoder_heads, decoder_heads;
    int encoder_ffn, decoder_ffn, max_position_embeddings, max_length, scale_embedding;
    int bos_token_id, pad_token_id, eos_token_id, decoder_start_token_id;
} orc_config;

typedef struct {
    int beam_size;       /* 1 = greedy */
    int max_new_tokens;  /* 0 = 2*len+16 (src/translator.rs:182) */
    float length_penalty;
    int sync_every;
} orc_gen_options;

typedef struct orc_model orc_model;
typedef struct orc_state orc_state;

const char *orc_last_error(void);
/* OpenMP threads a parallel region of the oracle uses (omp_get_max_threads). */
int orc_threads(void);
float orc_h2f(uint16_t h);
uint16_t orc_f2h(float f);
int orc_type_block(uint32_t type, int *block_elems, int *block_bytes);
int orc_dequant(uint32_t type, const void *src, int64_t n, float *y);
int orc_gemv(uint32_t type, const void *w, int N, int K, const float *x, int rows, float *y);
void orc_sinusoidal_table(int n, int dim, int padding_idx, float *out);

orc_model *orc_load(const char *gguf_path);
void orc_free(orc_model *m);
void orc_get_config(const orc_model *m, orc_config *out);
orc_state *orc_encode(const orc_model *m, const uint32_t *ids, const uint32_t *lens, int b, int max_new, int flags,
                      float *enc_out);
void orc_state_free(orc_state *st);
int orc_decode(const orc_model *m, orc_state *st, const uint32_t *ids, int t, float *logits, float *hidden);
int orc_generate(const orc_model *m, const uint32_t *ids, const uint32_t *lens, int b, uint32_t tgt_lang,
                 const orc_gen_options *o, int flags, uint32_t *out, int out_cap, int *out_len, float *min_gap);

/* Beam search (src/translator.rs:250-335) over a scripted decoder: fn fills
 * logprobs[rows][V] given each row's history hist[rows][hist_len] (the tokens fed after
 * [decoder_start, tgt_lang], reordered with the row); step is 1-based.  mutant != 0
 * plants one of the oracle's numbered mistakes (tests only).  out is [b][max_new]. */
typedef int (*orc_script_fn)(void *user, int step, int rows, const uint32_t *hist, int hist_len, float *logprobs);
int orc_beam_scripted(int b, int k, int V, uint32_t eos, int max_new, float length_penalty, int flags,
                      orc_script_fn fn, void *user, int mutant, uint32_t *out, int *ntok);

#ifdef __cplusplus
}
#endif
#endif
