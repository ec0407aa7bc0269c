/*
 * oracle.c -- CPU restatement of malaga's *dequantized* NLLB/M2M100 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * product path and the timed CPU baseline of bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library (malaga_amd/) never links, loads or calls it.
 *
 * What it restates (reference = /root/reference/crates/malaga-core):
 *   - GGUF v3 container parsing (candle gguf_file; keys/names from
 *     src/config.rs:71-116 and src/convert.rs:214-318)
 *   - ggml block dequantization: F32, F16, BF16, Q8_0, Q4_K, Q5_K, Q6_K
 *     (candle-core 0.11 k_quants, which follows ggml's public block formats;
 *     the crate is not vendored, see tests/test_oracle_blocks.py for the
 *     closed-form and hand-built-block checks that pin these)
 *   - sinusoidal position table (src/model.rs:324-340, computed in f64)
 *   - encoder + cross K/V projection (src/model.rs:145-153, 460-500)
 *   - generic decoder step with KV cache (src/model.rs:101-109, 118-189,
 *     514-540); optional f16 rounding of self/cross K/V as the fused path
 *     stores them (kernels/malaga.cu:142-154, src/graph.rs:94-97)
 *   - greedy decoding (src/translator.rs:214-241), beam search
 *     (src/translator.rs:250-358), the per-row budget and truncation of
 *     generate_to (src/translator.rs:175-207)
 *
 * Arithmetic: activations are stored as f32 between ops, like the reference;
 * every dot product and reduction accumulates in f64, so the oracle sits
 * closer to the exact value of the dequantized path than any f32 kernel.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <omp.h>

#include "oracle.h"

/* ------------------------------------------------------------------ f16 */

float orc_h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f;
    const uint32_t m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else { /* subnormal: m * 2^-24 */
            float f = (float)m * (1.0f / 16777216.0f);
            memcpy(&bits, &f, 4);
            bits |= s;
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* IEEE binary32 -> binary16, round to nearest even (what __float2half does). */
uint16_t orc_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                                    /* below the f16 normal range */
        /* value = ax_float; result = round(value * 2^24) as subnormal integer */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
        const uint32_t e = ax >> 23, mant = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e; /* value = mant * 2^(e-150); want * 2^24 */
        uint32_t q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ax - 0x38000000u; /* rebias exponent 127 -> 15 (in the high bits) */
    const uint32_t lo = r & 0x1fffu;
    r >>= 13;
    if (lo > 0x1000u || (lo == 0x1000u && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

static inline float round_f16(float f) { return orc_h2f(orc_f2h(f)); }

static inline float bf16_to_f32(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* -------------------------------------------------------- block formats */
/* ggml type ids and block geometry (public GGUF spec). */
enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30 };

int orc_type_block(uint32_t t, int *block_elems, int *block_bytes) {
    switch (t) {
    case T_F32: *block_elems = 1; *block_bytes = 4; return 0;
    case T_F16: *block_elems = 1; *block_bytes = 2; return 0;
    case T_BF16: *block_elems = 1; *block_bytes = 2; return 0;
    case T_Q8_0: *block_elems = 32; *block_bytes = 34; return 0;
    case T_Q4_K: *block_elems = 256; *block_bytes = 144; return 0;
    case T_Q5_K: *block_elems = 256; *block_bytes = 176; return 0;
    case T_Q6_K: *block_elems = 256; *block_bytes = 210; return 0;
    default: return -1;
    }
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* 6-bit scale/min pair j (0..7) of a Q4_K/Q5_K block's 12-byte table. */
static void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* Dequantizes n elements (n multiple of the block size) of type t. */
int orc_dequant(uint32_t t, const void *src, int64_t n, float *y) {
    const uint8_t *p = (const uint8_t *)src;
    switch (t) {
    case T_F32: memcpy(y, src, (size_t)n * 4); return 0;
    case T_F16: for (int64_t i = 0; i < n; ++i) y[i] = orc_h2f(rd16(p + 2 * i)); return 0;
    case T_BF16: for (int64_t i = 0; i < n; ++i) y[i] = bf16_to_f32(rd16(p + 2 * i)); return 0;
    case T_Q8_0:
        if (n % 32) return -1;
        for (int64_t b = 0; b < n / 32; ++b, p += 34) {
            const float d = orc_h2f(rd16(p));
            for (int l = 0; l < 32; ++l) *y++ = d * (float)(int8_t)p[2 + l];
        }
        return 0;
    case T_Q4_K:
        if (n % 256) return -1;
        for (int64_t b = 0; b < n / 256; ++b, p += 144) {
            const float d = orc_h2f(rd16(p)), dmin = orc_h2f(rd16(p + 2));
            const uint8_t *sc = p + 4, *q = p + 16;
            for (int g = 0; g < 4; ++g, q += 32) {
                int s0, m0, s1, m1;
                scale_min_k4(2 * g, sc, &s0, &m0);
                scale_min_k4(2 * g + 1, sc, &s1, &m1);
                const float d0 = d * s0, mm0 = dmin * m0, d1 = d * s1, mm1 = dmin * m1;
                for (int l = 0; l < 32; ++l) y[l] = d0 * (q[l] & 0xF) - mm0;
                for (int l = 0; l < 32; ++l) y[32 + l] = d1 * (q[l] >> 4) - mm1;
                y += 64;
            }
        }
        return 0;
    case T_Q5_K:
        if (n % 256) return -1;
        for (int64_t b = 0; b < n / 256; ++b, p += 176) {
            const float d = orc_h2f(rd16(p)), dmin = orc_h2f(rd16(p + 2));
            const uint8_t *sc = p + 4, *qh = p + 16, *ql = p + 48;
            for (int g = 0; g < 4; ++g, ql += 32) {
                int s0, m0, s1, m1;
                scale_min_k4(2 * g, sc, &s0, &m0);
                scale_min_k4(2 * g + 1, sc, &s1, &m1);
                const float d0 = d * s0, mm0 = dmin * m0, d1 = d * s1, mm1 = dmin * m1;
                for (int l = 0; l < 32; ++l) y[l] = d0 * ((ql[l] & 0xF) + (((qh[l] >> (2 * g)) & 1) << 4)) - mm0;
                for (int l = 0; l < 32; ++l) y[32 + l] = d1 * ((ql[l] >> 4) + (((qh[l] >> (2 * g + 1)) & 1) << 4)) - mm1;
                y += 64;
            }
        }
        return 0;
    case T_Q6_K:
        if (n % 256) return -1;
        for (int64_t b = 0; b < n / 256; ++b, p += 210) {
            const uint8_t *ql = p, *qh = p + 128;
            const int8_t *sc = (const int8_t *)(p + 192);
            const float d = orc_h2f(rd16(p + 208));
            for (int half = 0; half < 2; ++half, ql += 64, qh += 32, sc += 8) {
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    y[l] = d * sc[is] * q1;
                    y[l + 32] = d * sc[is + 2] * q2;
                    y[l + 64] = d * sc[is + 4] * q3;
                    y[l + 96] = d * sc[is + 6] * q4;
                }
                y += 128;
            }
        }
        return 0;
    default: return -1;
    }
}

/* ---------------------------------------------------------------- GGUF */

typedef struct {
    char name[96];
    uint32_t type;
    int ndims;
    uint64_t ne[4];
    uint64_t offset;
} gg_tensor;

typedef struct {
    char key[96];
    uint32_t type;
    uint64_t u;  /* integer / bool value */
    double f;    /* float value */
    const char *str; /* string value (not terminated) */
    uint64_t slen;
} gg_kv;

typedef struct {
    uint8_t *map;
    size_t size;
    int n_tensors, n_kv;
    gg_tensor *t;
    gg_kv *kv;
    const uint8_t *data;
} gguf;

typedef struct {
    const uint8_t *p, *end;
    int err;
} rdr;

static uint64_t rd_u(rdr *r, int n) {
    if (r->p + n > r->end) { r->err = 1; return 0; }
    uint64_t v = 0;
    for (int i = 0; i < n; ++i) v |= (uint64_t)r->p[i] << (8 * i);
    r->p += n;
    return v;
}

static const char *rd_str(rdr *r, uint64_t *len) {
    *len = rd_u(r, 8);
    if (r->err || r->p + *len > r->end) { r->err = 1; return NULL; }
    const char *s = (const char *)r->p;
    r->p += *len;
    return s;
}

static int scalar_size(uint32_t vt) {
    switch (vt) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return -1;
    }
}

static void skip_value(rdr *r, uint32_t vt) {
    if (vt == 8) { uint64_t l; rd_str(r, &l); return; }
    if (vt == 9) {
        const uint32_t et = (uint32_t)rd_u(r, 4);
        const uint64_t n = rd_u(r, 8);
        for (uint64_t i = 0; i < n && !r->err; ++i) skip_value(r, et);
        return;
    }
    const int s = scalar_size(vt);
    if (s < 0 || r->p + s > r->end) { r->err = 1; return; }
    r->p += s;
}

static void gguf_close(gguf *g) {
    if (g->map) munmap(g->map, g->size);
    free(g->t);
    free(g->kv);
    memset(g, 0, sizeof(*g));
}

static int gguf_open(const char *path, gguf *g) {
    memset(g, 0, sizeof(*g));
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return -1;
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return -1; }
    g->size = (size_t)st.st_size;
    g->map = mmap(NULL, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (g->map == MAP_FAILED) { g->map = NULL; return -1; }
    rdr r = {g->map, g->map + g->size, 0};
    if (rd_u(&r, 4) != 0x46554747u) { gguf_close(g); return -2; }
    const uint32_t version = (uint32_t)rd_u(&r, 4);
    if (version < 2 || version > 3) { gguf_close(g); return -2; }
    g->n_tensors = (int)rd_u(&r, 8);
    g->n_kv = (int)rd_u(&r, 8);
    g->kv = calloc((size_t)g->n_kv + 1, sizeof(gg_kv));
    g->t = calloc((size_t)g->n_tensors + 1, sizeof(gg_tensor));
    uint64_t align = 32;
    for (int i = 0; i < g->n_kv && !r.err; ++i) {
        gg_kv *kv = &g->kv[i];
        uint64_t kl;
        const char *k = rd_str(&r, &kl);
        if (r.err) break;
        snprintf(kv->key, sizeof kv->key, "%.*s", (int)kl, k);
        kv->type = (uint32_t)rd_u(&r, 4);
        switch (kv->type) {
        case 0: case 7: kv->u = rd_u(&r, 1); break;
        case 1: kv->u = (uint64_t)(int64_t)(int8_t)rd_u(&r, 1); break;
        case 2: kv->u = rd_u(&r, 2); break;
        case 3: kv->u = (uint64_t)(int64_t)(int16_t)rd_u(&r, 2); break;
        case 4: kv->u = rd_u(&r, 4); break;
        case 5: kv->u = (uint64_t)(int64_t)(int32_t)rd_u(&r, 4); break;
        case 6: { uint32_t b = (uint32_t)rd_u(&r, 4); float f; memcpy(&f, &b, 4); kv->f = f; break; }
        case 10: case 11: kv->u = rd_u(&r, 8); break;
        case 12: { uint64_t b = rd_u(&r, 8); memcpy(&kv->f, &b, 8); break; }
        case 8: kv->str = rd_str(&r, &kv->slen); break;
        case 9: skip_value(&r, 9); break; /* arrays are not needed by the oracle */
        default: r.err = 1;
        }
        if (!strcmp(kv->key, "general.alignment") && kv->u) align = kv->u;
    }
    for (int i = 0; i < g->n_tensors && !r.err; ++i) {
        gg_tensor *t = &g->t[i];
        uint64_t nl;
        const char *n = rd_str(&r, &nl);
        if (r.err) break;
        snprintf(t->name, sizeof t->name, "%.*s", (int)nl, n);
        t->ndims = (int)rd_u(&r, 4);
        if (t->ndims < 1 || t->ndims > 4) { r.err = 1; break; }
        for (int d = 0; d < t->ndims; ++d) t->ne[d] = rd_u(&r, 8);
        t->type = (uint32_t)rd_u(&r, 4);
        t->offset = rd_u(&r, 8);
    }
    if (r.err) { gguf_close(g); return -2; }
    size_t pos = (size_t)(r.p - g->map);
    pos = (pos + align - 1) / align * align;
    g->data = g->map + pos;
    return 0;
}

static const gg_kv *gguf_kv(const gguf *g, const char *key) {
    for (int i = 0; i < g->n_kv; ++i)
        if (!strcmp(g->kv[i].key, key)) return &g->kv[i];
    return NULL;
}

static const gg_tensor *gguf_tensor(const gguf *g, const char *name) {
    for (int i = 0; i < g->n_tensors; ++i)
        if (!strcmp(g->t[i].name, name)) return &g->t[i];
    return NULL;
}

/* --------------------------------------------------------------- model */

typedef struct { float *w, *b; int n, k; } lin; /* w: [n][k] row-major, y = x w^T + b */
typedef struct { float *g, *b; } lnorm;
typedef struct { lnorm attn_norm, ffn_norm; lin qkv, out, up, down; } enc_layer;
typedef struct { lnorm attn_norm, cross_norm, ffn_norm; lin qkv, out, cross_q, cross_kv, cross_out, up, down; } dec_layer;

struct orc_model {
    orc_config cfg;
    float *embed; /* [vocab][d] */
    float *pos;   /* [max_pos + pad + 1][d] */
    int n_pos;
    float embed_scale;
    enc_layer *enc;
    dec_layer *dec;
    lnorm enc_norm, dec_norm;
    char err[256];
};

static char g_err[256];
const char *orc_last_error(void) { return g_err; }

int orc_threads(void) { return omp_get_max_threads(); }

static float *load_tensor(const gguf *g, const char *name, int64_t expect_n, int64_t expect_k) {
    const gg_tensor *t = gguf_tensor(g, name);
    if (!t) { snprintf(g_err, sizeof g_err, "missing tensor %s", name); return NULL; }
    int64_t n = 1;
    for (int d = 0; d < t->ndims; ++d) n *= (int64_t)t->ne[d];
    if ((int64_t)t->ne[0] != expect_k || n != expect_n * expect_k) {
        snprintf(g_err, sizeof g_err, "tensor %s has shape ne0=%llu n=%lld, expected [%lld, %lld]", name,
                 (unsigned long long)t->ne[0], (long long)n, (long long)expect_n, (long long)expect_k);
        return NULL;
    }
    int be, bb;
    if (orc_type_block(t->type, &be, &bb)) { snprintf(g_err, sizeof g_err, "tensor %s: unsupported type %u", name, t->type); return NULL; }
    float *y = malloc((size_t)n * sizeof(float));
    if (!y) { snprintf(g_err, sizeof g_err, "out of memory"); return NULL; }
    const int64_t rows = n / expect_k, row_bytes = expect_k / be * bb;
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(| : bad)
    for (int64_t r = 0; r < rows; ++r)
        bad |= orc_dequant(t->type, g->data + t->offset + r * row_bytes, expect_k, y + r * expect_k) != 0;
    if (bad) { free(y); snprintf(g_err, sizeof g_err, "tensor %s: bad row length", name); return NULL; }
    return y;
}

static int load_lin(const gguf *g, const char *p, int n, int k, lin *l) {
    char nm[128];
    snprintf(nm, sizeof nm, "%s.weight", p);
    l->w = load_tensor(g, nm, n, k);
    snprintf(nm, sizeof nm, "%s.bias", p);
    l->b = l->w ? load_tensor(g, nm, 1, n) : NULL;
    l->n = n;
    l->k = k;
    return l->w && l->b ? 0 : -1;
}

static int load_ln(const gguf *g, const char *p, int d, lnorm *l) {
    char nm[128];
    snprintf(nm, sizeof nm, "%s.weight", p);
    l->g = load_tensor(g, nm, 1, d);
    snprintf(nm, sizeof nm, "%s.bias", p);
    l->b = l->g ? load_tensor(g, nm, 1, d) : NULL;
    return l->g && l->b ? 0 : -1;
}

/* src/model.rs:324-340 (fairseq / M2M100 table, computed in f64, row pad zeroed) */
void orc_sinusoidal_table(int n, int dim, int padding_idx, float *out) {
    const int half = dim / 2;
    const double step = log(10000.0) / ((double)half - 1.0);
    memset(out, 0, (size_t)n * dim * sizeof(float));
    for (int p = 0; p < n; ++p) {
        if (p == padding_idx) continue;
        for (int i = 0; i < half; ++i) {
            const double a = (double)p * exp(-(double)i * step);
            out[(size_t)p * dim + i] = (float)sin(a);
            out[(size_t)p * dim + half + i] = (float)cos(a);
        }
    }
}

static int kv_u32(const gguf *g, const char *key, int *out) {
    const gg_kv *kv = gguf_kv(g, key);
    if (!kv || kv->type == 8 || kv->type == 9 || kv->type == 6 || kv->type == 12) {
        snprintf(g_err, sizeof g_err, "missing GGUF metadata key '%s'", key);
        return -1;
    }
    *out = (int)kv->u;
    return 0;
}

void orc_free(orc_model *m) {
    if (!m) return;
    free(m->embed);
    free(m->pos);
    if (m->enc)
        for (int i = 0; i < m->cfg.encoder_layers; ++i) {
            enc_layer *l = &m->enc[i];
            free(l->attn_norm.g); free(l->attn_norm.b); free(l->ffn_norm.g); free(l->ffn_norm.b);
            free(l->qkv.w); free(l->qkv.b); free(l->out.w); free(l->out.b);
            free(l->up.w); free(l->up.b); free(l->down.w); free(l->down.b);
        }
    if (m->dec)
        for (int i = 0; i < m->cfg.decoder_layers; ++i) {
            dec_layer *l = &m->dec[i];
            free(l->attn_norm.g); free(l->attn_norm.b); free(l->cross_norm.g); free(l->cross_norm.b);
            free(l->ffn_norm.g); free(l->ffn_norm.b);
            lin *ls[] = {&l->qkv, &l->out, &l->cross_q, &l->cross_kv, &l->cross_out, &l->up, &l->down};
            for (int j = 0; j < 7; ++j) { free(ls[j]->w); free(ls[j]->b); }
        }
    free(m->enc);
    free(m->dec);
    free(m->enc_norm.g); free(m->enc_norm.b); free(m->dec_norm.g); free(m->dec_norm.b);
    free(m);
}

/* src/config.rs:93-116 (keys), src/model.rs:343-433 (tensor names) */
orc_model *orc_load(const char *path) {
    gguf g;
    const int rc = gguf_open(path, &g);
    if (rc) { snprintf(g_err, sizeof g_err, "cannot read GGUF %s (%d)", path, rc); return NULL; }
    orc_model *m = calloc(1, sizeof(orc_model));
    orc_config *c = &m->cfg;
    const gg_kv *arch = gguf_kv(&g, "general.architecture");
    if (!arch || arch->type != 8 || arch->slen != 4 || memcmp(arch->str, "nllb", 4)) {
        snprintf(g_err, sizeof g_err, "unsupported architecture, expected 'nllb'");
        goto fail;
    }
    if (kv_u32(&g, "nllb.vocab_size", &c->vocab_size) || kv_u32(&g, "nllb.embedding_length", &c->d_model) ||
        kv_u32(&g, "nllb.encoder.block_count", &c->encoder_layers) ||
        kv_u32(&g, "nllb.decoder.block_count", &c->decoder_layers) ||
        kv_u32(&g, "nllb.encoder.attention.head_count", &c->encoder_heads) ||
        kv_u32(&g, "nllb.decoder.attention.head_count", &c->decoder_heads) ||
        kv_u32(&g, "nllb.encoder.feed_forward_length", &c->encoder_ffn) ||
        kv_u32(&g, "nllb.decoder.feed_forward_length", &c->decoder_ffn) ||
        kv_u32(&g, "nllb.context_length", &c->max_position_embeddings) ||
        kv_u32(&g, "nllb.max_length", &c->max_length) || kv_u32(&g, "nllb.scale_embedding", &c->scale_embedding) ||
        kv_u32(&g, "tokenizer.ggml.bos_token_id", &c->bos_token_id) ||
        kv_u32(&g, "tokenizer.ggml.padding_token_id", &c->pad_token_id) ||
        kv_u32(&g, "tokenizer.ggml.eos_token_id", &c->eos_token_id) ||
        kv_u32(&g, "tokenizer.ggml.decoder_start_token_id", &c->decoder_start_token_id))
        goto fail;
    const int d = c->d_model, V = c->vocab_size;
    if (!(m->embed = load_tensor(&g, "token_embd.weight", V, d))) goto fail;
    m->n_pos = c->max_position_embeddings + c->pad_token_id + 1;
    m->pos = malloc((size_t)m->n_pos * d * sizeof(float));
    orc_sinusoidal_table(m->n_pos, d, c->pad_token_id, m->pos);
    m->embed_scale = c->scale_embedding ? (float)sqrt((double)d) : 1.0f;
    m->enc = calloc((size_t)c->encoder_layers, sizeof(enc_layer));
    m->dec = calloc((size_t)c->decoder_layers, sizeof(dec_layer));
    char p[96];
    for (int i = 0; i < c->encoder_layers; ++i) {
        enc_layer *l = &m->enc[i];
        const int f = c->encoder_ffn;
#define E(s) (snprintf(p, sizeof p, "enc.blk.%d." s, i), p)
        if (load_ln(&g, E("attn_norm"), d, &l->attn_norm) || load_lin(&g, E("attn_qkv"), 3 * d, d, &l->qkv) ||
            load_lin(&g, E("attn_out"), d, d, &l->out) || load_ln(&g, E("ffn_norm"), d, &l->ffn_norm) ||
            load_lin(&g, E("ffn_up"), f, d, &l->up) || load_lin(&g, E("ffn_down"), d, f, &l->down))
            goto fail;
#undef E
    }
    for (int i = 0; i < c->decoder_layers; ++i) {
        dec_layer *l = &m->dec[i];
        const int f = c->decoder_ffn;
#define D(s) (snprintf(p, sizeof p, "dec.blk.%d." s, i), p)
        if (load_ln(&g, D("attn_norm"), d, &l->attn_norm) || load_lin(&g, D("attn_qkv"), 3 * d, d, &l->qkv) ||
            load_lin(&g, D("attn_out"), d, d, &l->out) || load_ln(&g, D("cross_attn_norm"), d, &l->cross_norm) ||
            load_lin(&g, D("cross_attn_q"), d, d, &l->cross_q) || load_lin(&g, D("cross_attn_kv"), 2 * d, d, &l->cross_kv) ||
            load_lin(&g, D("cross_attn_out"), d, d, &l->cross_out) || load_ln(&g, D("ffn_norm"), d, &l->ffn_norm) ||
            load_lin(&g, D("ffn_up"), f, d, &l->up) || load_lin(&g, D("ffn_down"), d, f, &l->down))
            goto fail;
#undef D
    }
    if (load_ln(&g, "enc.output_norm", d, &m->enc_norm) || load_ln(&g, "dec.output_norm", d, &m->dec_norm)) goto fail;
    gguf_close(&g);
    return m;
fail:
    gguf_close(&g);
    orc_free(m);
    return NULL;
}

void orc_get_config(const orc_model *m, orc_config *out) { *out = m->cfg; }

/* ----------------------------------------------------------- primitives */

/* y[r][n] = f32(sum_k x[r][k] w[n][k]) (+ b[n]).  Every sum starts at 0 and adds the
 * products in k order in f64; a product of two floats is exact in f64, so each step
 * rounds once whether or not it is fused.  Layout for speed only: the input rows are
 * interleaved in blocks of 8 (xt[blk][k][8]), so one weight load serves 8 independent
 * sums held in two 4-wide f64 vectors, and weight rows are the outer loop, so a batch
 * reads every weight once. */
typedef double orc_v4d __attribute__((vector_size(32)));
typedef float orc_v4f __attribute__((vector_size(16)));

/* acc[i][j] = sum_k xt[k][j] w_i[k] for 4 weight rows w_0..w_3 (8 independent chains). */
__attribute__((target_clones("avx512f", "avx2", "default")))
static void dot4x8(const float *xt, const float *w0, const float *w1, const float *w2, const float *w3, int K,
                   double *acc) {
    orc_v4d a0 = {0, 0, 0, 0}, a1 = a0, a2 = a0, a3 = a0, a4 = a0, a5 = a0, a6 = a0, a7 = a0;
    for (int k = 0; k < K; ++k) {
        orc_v4f lo, hi;
        memcpy(&lo, xt + (size_t)k * 8, 16);
        memcpy(&hi, xt + (size_t)k * 8 + 4, 16);
        const orc_v4d xl = __builtin_convertvector(lo, orc_v4d), xh = __builtin_convertvector(hi, orc_v4d);
        const double q0 = w0[k], q1 = w1[k], q2 = w2[k], q3 = w3[k];
        const orc_v4d v0 = {q0, q0, q0, q0}, v1 = {q1, q1, q1, q1}, v2 = {q2, q2, q2, q2}, v3 = {q3, q3, q3, q3};
        a0 += xl * v0;
        a1 += xh * v0;
        a2 += xl * v1;
        a3 += xh * v1;
        a4 += xl * v2;
        a5 += xh * v2;
        a6 += xl * v3;
        a7 += xh * v3;
    }
    memcpy(acc, &a0, 32);
    memcpy(acc + 4, &a1, 32);
    memcpy(acc + 8, &a2, 32);
    memcpy(acc + 12, &a3, 32);
    memcpy(acc + 16, &a4, 32);
    memcpy(acc + 20, &a5, 32);
    memcpy(acc + 24, &a6, 32);
    memcpy(acc + 28, &a7, 32);
}

static void dot_rows(const float *x, int rows, const float *w, int N, int K, const float *bias, float *y) {
    const int nblk = (rows + 7) / 8;
    float *xt = calloc((size_t)nblk * K * 8, sizeof(float));
    for (int r = 0; r < rows; ++r)
        for (int k = 0; k < K; ++k) xt[((size_t)(r / 8) * K + k) * 8 + r % 8] = x[(size_t)r * K + k];
    /* row blocks in chunks of ~256 KB of xt, so a chunk stays in cache while the
     * weight rows stream past it */
    int chunk = (int)(262144 / ((size_t)K * 32));
    if (chunk < 1) chunk = 1;
    for (int b0 = 0; b0 < nblk; b0 += chunk) {
        const int b1 = b0 + chunk < nblk ? b0 + chunk : nblk;
#pragma omp parallel for schedule(static)
        for (int n0 = 0; n0 < N; n0 += 4) {
            const float *wr[4];
            for (int i = 0; i < 4; ++i) wr[i] = w + (size_t)(n0 + i < N ? n0 + i : n0) * K;
            for (int blk = b0; blk < b1; ++blk) {
                double acc[32];
                dot4x8(xt + (size_t)blk * K * 8, wr[0], wr[1], wr[2], wr[3], K, acc);
                for (int i = 0; i < 4 && n0 + i < N; ++i)
                    for (int j = 0; j < 8 && blk * 8 + j < rows; ++j) {
                        const float v = (float)acc[i * 8 + j];
                        y[(size_t)(blk * 8 + j) * N + n0 + i] = bias ? v + bias[n0 + i] : v;
                    }
            }
        }
    }
    free(xt);
}

/* QMatMul then broadcast_add (src/model.rs:80-84) */
static void linear(const float *x, int rows, const lin *l, float *y) { dot_rows(x, rows, l->w, l->n, l->k, l->b, y); }

/* candle_nn LayerNorm, eps = 1e-5 (src/config.rs:58): biased variance. */
static void layer_norm(const float *x, int rows, int d, const lnorm *l, float *y) {
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (size_t)r * d;
        double s = 0, s2 = 0;
        for (int i = 0; i < d; ++i) s += xr[i];
        const double mean = s / d;
        for (int i = 0; i < d; ++i) s2 += (xr[i] - mean) * (xr[i] - mean);
        const double rstd = 1.0 / sqrt(s2 / d + 1e-5);
        for (int i = 0; i < d; ++i) y[(size_t)r * d + i] = (float)((xr[i] - mean) * rstd * l->g[i] + l->b[i]);
    }
}

/* softmax(q k^T + mask) v for one (row, head); keys j >= nvalid (or masked by the
 * causal limit) contribute exp(-inf) = 0, exactly as the additive -inf masks of
 * src/model.rs:101-109, 480-500, 520-528. */
static void attend(const float *q, const float *K, const float *V, int L, int hd, int nvalid, float *out) {
    double *sc = malloc((size_t)(L > 0 ? L : 1) * sizeof(double));
    double mx = -INFINITY;
    for (int j = 0; j < nvalid; ++j) {
        double a = 0;
        for (int e = 0; e < hd; ++e) a += (double)q[e] * K[(size_t)j * hd + e];
        sc[j] = (float)a; /* scores are an f32 tensor in the reference */
        if (sc[j] > mx) mx = sc[j];
    }
    double sum = 0;
    for (int j = 0; j < nvalid; ++j) { sc[j] = exp(sc[j] - mx); sum += sc[j]; }
    for (int e = 0; e < hd; ++e) {
        double a = 0;
        for (int j = 0; j < nvalid; ++j) a += sc[j] * V[(size_t)j * hd + e];
        out[e] = (float)(a / sum);
    }
    free(sc);
}

/* ------------------------------------------------------------- encoder */

struct orc_state {
    int b, s, H, hd, d, max_len, pos, layers;
    uint32_t *lens;
    float **ck, **cv; /* per decoder layer: [b][H][s][hd] */
    float **kc, **vc; /* per decoder layer: [b][H][max_len][hd] */
    int kv_f16;
};

void orc_state_free(orc_state *st) {
    if (!st) return;
    for (int i = 0; i < st->layers; ++i) { free(st->ck[i]); free(st->cv[i]); free(st->kc[i]); free(st->vc[i]); }
    free(st->ck); free(st->cv); free(st->kc); free(st->vc); free(st->lens);
    free(st);
}

/* src/model.rs:463-500 (+ 503-512 for the cache size max_new + 2).
 * enc_out, if not NULL, receives the normalized encoder output [b][s][d]. */
orc_state *orc_encode(const orc_model *m, const uint32_t *ids, const uint32_t *lens, int b, int max_new, int flags,
                      float *enc_out) {
    const orc_config *c = &m->cfg;
    const int d = c->d_model, H = c->encoder_heads, hd = d / H;
    int s = 0;
    for (int i = 0; i < b; ++i) if ((int)lens[i] > s) s = (int)lens[i];
    if (b <= 0 || s <= 0) { snprintf(g_err, sizeof g_err, "empty batch"); return NULL; }
    const int n = b * s;
    float *x = calloc((size_t)n * d, 4), *h = calloc((size_t)n * d, 4), *qkv = calloc((size_t)n * 3 * d, 4);
    float *att = calloc((size_t)n * d, 4), *y = calloc((size_t)n * d, 4);
    const int f = c->encoder_ffn;
    float *u = calloc((size_t)n * (f > 2 * d ? f : 2 * d), 4);
    /* embedding * scale + positions (pad_batch: pads use token pad, position pad) */
    size_t off = 0;
    for (int i = 0; i < b; ++i) {
        for (int j = 0; j < s; ++j) {
            const int valid = j < (int)lens[i];
            const uint32_t tok = valid ? ids[off + j] : (uint32_t)c->pad_token_id;
            const uint32_t p = valid ? (uint32_t)(j + c->pad_token_id + 1) : (uint32_t)c->pad_token_id;
            const float *e = m->embed + (size_t)tok * d, *pe = m->pos + (size_t)p * d;
            for (int k = 0; k < d; ++k) x[((size_t)i * s + j) * d + k] = e[k] * m->embed_scale + pe[k];
        }
        off += lens[i];
    }
    for (int li = 0; li < c->encoder_layers; ++li) {
        const enc_layer *l = &m->enc[li];
        layer_norm(x, n, d, &l->attn_norm, h);
        linear(h, n, &l->qkv, qkv);
#pragma omp parallel for collapse(2) schedule(static)
        for (int i = 0; i < b; ++i)
            for (int hh = 0; hh < H; ++hh) {
                float *K = malloc((size_t)s * hd * 4), *V = malloc((size_t)s * hd * 4);
                for (int j = 0; j < s; ++j)
                    for (int e = 0; e < hd; ++e) {
                        K[j * hd + e] = qkv[((size_t)i * s + j) * 3 * d + d + hh * hd + e];
                        V[j * hd + e] = qkv[((size_t)i * s + j) * 3 * d + 2 * d + hh * hd + e];
                    }
                for (int t = 0; t < s; ++t)
                    attend(qkv + ((size_t)i * s + t) * 3 * d + hh * hd, K, V, s, hd, (int)lens[i],
                           att + ((size_t)i * s + t) * d + hh * hd);
                free(K); free(V);
            }
        linear(att, n, &l->out, y);
        for (size_t k = 0; k < (size_t)n * d; ++k) x[k] = x[k] + y[k];
        layer_norm(x, n, d, &l->ffn_norm, h);
        linear(h, n, &l->up, u);
        for (size_t k = 0; k < (size_t)n * f; ++k) u[k] = u[k] > 0 ? u[k] : 0;
        linear(u, n, &l->down, y);
        for (size_t k = 0; k < (size_t)n * d; ++k) x[k] = x[k] + y[k];
    }
    layer_norm(x, n, d, &m->enc_norm, h);
    if (enc_out) memcpy(enc_out, h, (size_t)n * d * 4);

    orc_state *st = calloc(1, sizeof(orc_state));
    const int Hd = c->decoder_heads, hdd = d / Hd, L = c->decoder_layers;
    st->b = b; st->s = s; st->H = Hd; st->hd = hdd; st->d = d; st->layers = L; st->pos = 0;
    st->max_len = max_new + 2;
    st->kv_f16 = (flags & ORC_KV_F16) != 0;
    st->lens = malloc((size_t)b * 4);
    memcpy(st->lens, lens, (size_t)b * 4);
    st->ck = calloc(L, sizeof(float *)); st->cv = calloc(L, sizeof(float *));
    st->kc = calloc(L, sizeof(float *)); st->vc = calloc(L, sizeof(float *));
    for (int li = 0; li < L; ++li) {
        linear(h, n, &m->dec[li].cross_kv, u); /* [n][2d] */
        st->ck[li] = malloc((size_t)b * Hd * s * hdd * 4);
        st->cv[li] = malloc((size_t)b * Hd * s * hdd * 4);
        st->kc[li] = calloc((size_t)b * Hd * st->max_len * hdd, 4);
        st->vc[li] = calloc((size_t)b * Hd * st->max_len * hdd, 4);
        for (int i = 0; i < b; ++i)
            for (int hh = 0; hh < Hd; ++hh)
                for (int j = 0; j < s; ++j)
                    for (int e = 0; e < hdd; ++e) {
                        const size_t src = ((size_t)i * s + j) * 2 * d + hh * hdd + e;
                        const size_t dst = (((size_t)i * Hd + hh) * s + j) * hdd + e;
                        float kk = u[src], vv = u[src + d];
                        if (st->kv_f16) { kk = round_f16(kk); vv = round_f16(vv); }
                        st->ck[li][dst] = kk;
                        st->cv[li][dst] = vv;
                    }
    }
    free(x); free(h); free(qkv); free(att); free(y); free(u);
    return st;
}

/* ------------------------------------------------------------- decoder */

/* src/model.rs:514-540: feeds ids [b][t] and writes the logits of the last
 * position [b][vocab] (and, if not NULL, the dec_norm'ed hidden state [b][d]). */
int orc_decode(const orc_model *m, orc_state *st, const uint32_t *ids, int t, float *logits, float *hidden) {
    const orc_config *c = &m->cfg;
    const int b = st->b, d = st->d, H = st->H, hd = st->hd, V = c->vocab_size;
    if (st->pos + t > st->max_len) { snprintf(g_err, sizeof g_err, "decoder cache overflow"); return -1; }
    if (st->pos + t + c->pad_token_id + 1 > m->n_pos) { snprintf(g_err, sizeof g_err, "position overflow"); return -1; }
    const int n = b * t, f = c->decoder_ffn;
    float *x = calloc((size_t)n * d, 4), *h = calloc((size_t)n * d, 4), *qkv = calloc((size_t)n * 3 * d, 4);
    float *att = calloc((size_t)n * d, 4), *y = calloc((size_t)n * d, 4), *u = calloc((size_t)n * f, 4);
    for (int i = 0; i < b; ++i)
        for (int j = 0; j < t; ++j) {
            const uint32_t tok = ids[i * t + j];
            if (tok >= (uint32_t)V) { snprintf(g_err, sizeof g_err, "token id out of range"); return -1; }
            const uint32_t p = (uint32_t)(st->pos + j + c->pad_token_id + 1);
            for (int k = 0; k < d; ++k)
                x[((size_t)i * t + j) * d + k] = m->embed[(size_t)tok * d + k] * m->embed_scale + m->pos[(size_t)p * d + k];
        }
    const int past = st->pos, ML = st->max_len, s = st->s;
    for (int li = 0; li < c->decoder_layers; ++li) {
        const dec_layer *l = &m->dec[li];
        layer_norm(x, n, d, &l->attn_norm, h);
        linear(h, n, &l->qkv, qkv);
        for (int i = 0; i < b; ++i)
            for (int j = 0; j < t; ++j)
                for (int hh = 0; hh < H; ++hh)
                    for (int e = 0; e < hd; ++e) {
                        const size_t src = ((size_t)i * t + j) * 3 * d + hh * hd + e;
                        const size_t dst = (((size_t)i * H + hh) * ML + past + j) * hd + e;
                        float kk = qkv[src + d], vv = qkv[src + 2 * d];
                        if (st->kv_f16) { kk = round_f16(kk); vv = round_f16(vv); }
                        st->kc[li][dst] = kk;
                        st->vc[li][dst] = vv;
                    }
#pragma omp parallel for collapse(3) schedule(static)
        for (int i = 0; i < b; ++i)
            for (int hh = 0; hh < H; ++hh)
                for (int j = 0; j < t; ++j) {
                    const size_t base = ((size_t)i * H + hh) * ML * hd;
                    attend(qkv + ((size_t)i * t + j) * 3 * d + hh * hd, st->kc[li] + base, st->vc[li] + base, ML, hd,
                           past + j + 1, att + ((size_t)i * t + j) * d + hh * hd);
                }
        linear(att, n, &l->out, y);
        for (size_t k = 0; k < (size_t)n * d; ++k) x[k] = x[k] + y[k];
        layer_norm(x, n, d, &l->cross_norm, h);
        linear(h, n, &l->cross_q, y);
#pragma omp parallel for collapse(3) schedule(static)
        for (int i = 0; i < b; ++i)
            for (int hh = 0; hh < H; ++hh)
                for (int j = 0; j < t; ++j) {
                    const size_t base = ((size_t)i * H + hh) * s * hd;
                    attend(y + ((size_t)i * t + j) * d + hh * hd, st->ck[li] + base, st->cv[li] + base, s, hd,
                           (int)st->lens[i], att + ((size_t)i * t + j) * d + hh * hd);
                }
        linear(att, n, &l->cross_out, y);
        for (size_t k = 0; k < (size_t)n * d; ++k) x[k] = x[k] + y[k];
        layer_norm(x, n, d, &l->ffn_norm, h);
        linear(h, n, &l->up, u);
        for (size_t k = 0; k < (size_t)n * f; ++k) u[k] = u[k] > 0 ? u[k] : 0;
        linear(u, n, &l->down, y);
        for (size_t k = 0; k < (size_t)n * d; ++k) x[k] = x[k] + y[k];
    }
    st->pos += t;
    /* lm_head(dec_norm(x[:, t-1])) with the tied embedding, src/model.rs:538-540 */
    float *last = malloc((size_t)b * d * 4);
    for (int i = 0; i < b; ++i) memcpy(last + (size_t)i * d, x + ((size_t)i * t + t - 1) * d, (size_t)d * 4);
    layer_norm(last, b, d, &m->dec_norm, h);
    if (hidden) memcpy(hidden, h, (size_t)b * d * 4);
    dot_rows(h, b, m->embed, V, d, NULL, logits);
    free(last); free(x); free(h); free(qkv); free(att); free(y); free(u);
    return 0;
}

/* Beam search reorders every cached tensor (src/model.rs:209-226). */
static int state_reorder(orc_state *st, const uint32_t *idx, int nb) {
    const size_t self_row = (size_t)st->H * st->max_len * st->hd, cross_row = (size_t)st->H * st->s * st->hd;
    for (int li = 0; li < st->layers; ++li) {
        float *a = malloc(nb * self_row * 4), *bb = malloc(nb * self_row * 4);
        float *c = malloc(nb * cross_row * 4), *dd = malloc(nb * cross_row * 4);
        for (int i = 0; i < nb; ++i) {
            memcpy(a + i * self_row, st->kc[li] + idx[i] * self_row, self_row * 4);
            memcpy(bb + i * self_row, st->vc[li] + idx[i] * self_row, self_row * 4);
            memcpy(c + i * cross_row, st->ck[li] + idx[i] * cross_row, cross_row * 4);
            memcpy(dd + i * cross_row, st->cv[li] + idx[i] * cross_row, cross_row * 4);
        }
        free(st->kc[li]); free(st->vc[li]); free(st->ck[li]); free(st->cv[li]);
        st->kc[li] = a; st->vc[li] = bb; st->ck[li] = c; st->cv[li] = dd;
    }
    uint32_t *lens = malloc((size_t)nb * 4);
    for (int i = 0; i < nb; ++i) lens[i] = st->lens[idx[i]];
    free(st->lens);
    st->lens = lens;
    st->b = nb;
    return 0;
}

/* ------------------------------------------------------------ decoding */

/* Argmax with ties to the lowest index (kernels/malaga.cu:258-265, 302-307).
 * Also reports the gap between the best and second-best logit. */
static uint32_t argmax_row(const float *x, int V, int mask_eos, uint32_t eos, float *gap) {
    float best = -INFINITY, second = -INFINITY;
    uint32_t bi = 0;
    int have = 0;
    for (int v = 0; v < V; ++v) {
        float a = x[v];
        if (mask_eos && (uint32_t)v == eos) a = -INFINITY;
        if (!have || a > best) {
            if (have) second = best > second ? best : second;
            best = a; bi = (uint32_t)v; have = 1;
        } else if (a > second) {
            second = a;
        }
    }
    if (gap) *gap = best - second;
    return bi;
}

static int budget(const orc_config *c, int len, int max_new_tokens) {
    int cap = c->max_length < c->max_position_embeddings - 2 ? c->max_length : c->max_position_embeddings - 2;
    int v = max_new_tokens > 0 ? max_new_tokens : 2 * len + 16;
    if (v < 1) v = 1;
    if (v > cap) v = cap;
    return v;
}

/* Shortlist decoding (src/model.rs:594-603, kernels/malaga.cu:229-243, 286-326): the
 * candidates of row r are the shortlist rows, then the row's source tokens, in that
 * order (argmax ties to the lowest position).  A shortlist row is token_embd's row for
 * its id and a source candidate is the token's own embedding, so each candidate's
 * logit is the full-vocabulary logit of its token.  Padding positions of the source
 * add the pad token, which every shortlist holds (ids 0..3), so they are not listed. */
typedef struct {
    const uint32_t *ids;  /* sorted shortlist, n >= 1 */
    int n;
    const uint32_t *src;  /* flattened source ids of the batch */
    const uint32_t *off;  /* [b + 1] row offsets into src */
} orc_shortlist;

static uint32_t argmax_shortlist(const float *x, const orc_shortlist *sl, int row, int mask_eos, uint32_t eos,
                                 float *gap) {
    float best = -INFINITY, second = -INFINITY;
    uint32_t bt = 0;
    int have = 0;
    const int ns = (int)(sl->off[row + 1] - sl->off[row]);
    for (int i = 0; i < sl->n + ns; ++i) {
        const uint32_t t = i < sl->n ? sl->ids[i] : sl->src[sl->off[row] + (i - sl->n)];
        float a = x[t];
        if (mask_eos && t == eos) a = -INFINITY;
        if (!have || a > best) {
            if (have && bt != t) second = best > second ? best : second;
            best = a; bt = t; have = 1;
        } else if (t != bt && a > second) {
            second = a;
        }
    }
    if (gap) *gap = best - second;
    return bt;
}

/* src/translator.rs:214-241 (sl: the shortlist path of the fused GraphCache step) */
static int greedy(const orc_model *m, orc_state *st, int b, uint32_t tgt, int max_new, int sync_every, int flags,
                  uint32_t *toks /* [b][max_new] */, int *ntok, float *min_gap, const orc_shortlist *sl) {
    const orc_config *c = &m->cfg;
    const int V = c->vocab_size;
    float *logits = malloc((size_t)b * V * 4);
    uint32_t *start = malloc((size_t)b * 2 * 4);
    for (int i = 0; i < b; ++i) { start[2 * i] = (uint32_t)c->decoder_start_token_id; start[2 * i + 1] = tgt; }
    int rc = orc_decode(m, st, start, 2, logits, NULL);
    free(start);
    uint8_t *fin = calloc((size_t)b, 1);
    uint32_t *next = malloc((size_t)b * 4);
    int steps = 0;
    for (int step = 1; rc == 0 && step <= max_new; ++step) {
        int all = 1;
        for (int i = 0; i < b; ++i) {
            float gap;
            const uint32_t a = sl ? argmax_shortlist(logits + (size_t)i * V, sl, i, flags & ORC_EOS_MASK,
                                                     (uint32_t)c->eos_token_id, &gap)
                                  : argmax_row(logits + (size_t)i * V, V, flags & ORC_EOS_MASK, (uint32_t)c->eos_token_id, &gap);
            if (!fin[i] && min_gap && gap < *min_gap) *min_gap = gap;
            next[i] = fin[i] ? (uint32_t)c->pad_token_id : a;
            fin[i] |= next[i] == (uint32_t)c->eos_token_id;
            all &= fin[i];
            toks[(size_t)i * max_new + step - 1] = next[i];
        }
        steps = step;
        if (step == max_new || (step % sync_every == 0 && all)) break;
        rc = orc_decode(m, st, next, 1, logits, NULL);
    }
    for (int i = 0; i < b; ++i) { /* strip: take_while != eos */
        int k = 0;
        while (k < steps && toks[(size_t)i * max_new + k] != (uint32_t)c->eos_token_id) ++k;
        ntok[i] = k;
    }
    free(fin); free(next); free(logits);
    return rc;
}

typedef struct { float score; int n; uint32_t *toks; } hyp;

/* Top-k by k argmax passes: ties to the lowest index (src/translator.rs:343-358). */
static void topk_row(const float *x, int V, int k, float *vals, uint32_t *idx) {
    for (int j = 0; j < k; ++j) {
        float best = -INFINITY;
        uint32_t bi = 0;
        int have = 0;
        for (int v = 0; v < V; ++v) {
            int taken = 0;
            for (int q = 0; q < j; ++q) taken |= idx[q] == (uint32_t)v;
            const float a = taken ? -INFINITY : x[v];
            if (!have || a > best) { best = a; bi = (uint32_t)v; have = 1; }
        }
        vals[j] = best;
        idx[j] = bi;
    }
}

/* candle_nn::ops::log_softmax: (x - max) - ln(sum exp(x - max)) */
static void log_softmax_row(const float *x, int V, float *y) {
    float mx = -INFINITY;
    for (int v = 0; v < V; ++v) if (x[v] > mx) mx = x[v];
    double s = 0;
    for (int v = 0; v < V; ++v) s += exp((double)(x[v] - mx));
    const float ls = (float)log(s);
    for (int v = 0; v < V; ++v) y[v] = (x[v] - mx) - ls;
}

/* f32::total_cmp's order as a signed integer key (negative values' magnitude bits flipped). */
static int32_t total_key(float f) {
    int32_t i;
    memcpy(&i, &f, 4);
    return i ^ (int32_t)((uint32_t)(i >> 31) >> 1);
}

/* sort_by(|a, c| c.0.total_cmp(&a.0)): descending under the total order */
static int cand_cmp_desc(float a, float b) {
    const int32_t x = total_key(a), y = total_key(b);
    return x > y ? -1 : (x < y ? 1 : 0);
}

/* The decoder seen by the beam merge: `first` decodes [start, tgt] on all b*k rows,
 * `advance` makes row r continue row reorder[r] (src/model.rs:209-226) and feeds it
 * next[r]; both write one row of `width` values per decoder row.  `normalize`: the
 * values are logits (log_softmax applied here, src/model.rs:615-617), otherwise they
 * are already log-probabilities (scripted tests). */
typedef struct {
    int (*first)(void *self, float *out);
    int (*advance)(void *self, const uint32_t *reorder, const uint32_t *next, float *out);
    void *self;
    int width, normalize;
} beam_decoder;

/* Planted mistakes for the tests that check the known answers can tell them apart
 * (0 = the reference's rules). */
enum {
    MUT_STOP_STRICT = 1,     /* best_done > best_alive instead of >= */
    MUT_ALIVE_PEN_STEP = 2,  /* best_alive / penalty(step) instead of penalty(step + 1) */
    MUT_PAD_TOKEN = 3,       /* padded rows fed token 1 (NLLB's pad id) instead of EOS */
    MUT_DONE_LEN = 4,        /* done score / penalty(tokens) instead of penalty(tokens + 1) */
    MUT_FIRST_MAX = 5,       /* final pick: first maximum instead of Iterator::max_by's last */
    MUT_NO_COUNT = 6,        /* stop without done.len() >= k */
    MUT_PAD_SCORE = 8,       /* padded hypotheses score 0 instead of -inf */
    MUT_PUSH_AFTER_DONE = 9  /* finished sentences keep collecting done hypotheses */
};

/* src/translator.rs:250-335 over any decoder. */
static int beam_core(int b, int k, int max_new, float lp, uint32_t eos, int mask_eos, const beam_decoder *dec,
                     int mutant, uint32_t *out /* [b][max_new] */, int *ntok) {
    const int W = dec->width;
    hyp *alive = calloc((size_t)b * k, sizeof(hyp));
    int *nalive = calloc((size_t)b, sizeof(int));
    int *ndone = calloc((size_t)b, sizeof(int)), *capdone = calloc((size_t)b, sizeof(int));
    hyp **dl = calloc((size_t)b, sizeof(hyp *));
    uint8_t *is_done = calloc((size_t)b, 1);
    for (int s = 0; s < b; ++s) { nalive[s] = 1; alive[s * k].score = 0; alive[s * k].n = 0; alive[s * k].toks = NULL; }
    float *logits = malloc((size_t)b * k * W * 4), *lsm = malloc((size_t)W * 4);
    int rc = dec->first(dec->self, logits);
    float *vals = malloc((size_t)b * k * k * 4);
    uint32_t *idx = malloc((size_t)b * k * k * 4), *reorder = malloc((size_t)b * k * 4), *next = malloc((size_t)b * k * 4);
    typedef struct { float score; int bi; uint32_t tok; } cand;
    cand *cands = malloc((size_t)k * k * sizeof(cand));
    hyp *new_alive = calloc((size_t)k, sizeof(hyp));
#define PEN(len) powf((float)((len) > 1 ? (len) : 1), lp)
    for (int step = 1; rc == 0 && step <= max_new; ++step) {
        for (int r = 0; r < b * k; ++r) {
            float *row = logits + (size_t)r * W;
            if (mask_eos) row[eos] = -INFINITY; /* benchmark-only fixed lengths */
            if (dec->normalize) log_softmax_row(row, W, lsm);
            else memcpy(lsm, row, (size_t)W * 4);
            topk_row(lsm, W, k, vals + (size_t)r * k, idx + (size_t)r * k);
        }
        int nr = 0;
        for (int s = 0; s < b; ++s) {
            int nc = 0;
            for (int bi = 0; bi < nalive[s]; ++bi) {
                const int row = s * k + bi;
                for (int j = 0; j < k; ++j) {
                    cands[nc].score = alive[s * k + bi].score + vals[(size_t)row * k + j];
                    cands[nc].bi = bi;
                    cands[nc].tok = idx[(size_t)row * k + j];
                    ++nc;
                }
            }
            for (int i = 1; i < nc; ++i) { /* stable insertion sort, descending */
                cand x = cands[i];
                int j = i - 1;
                while (j >= 0 && cand_cmp_desc(cands[j].score, x.score) > 0) { cands[j + 1] = cands[j]; --j; }
                cands[j + 1] = x;
            }
            int na = 0;
            for (int ci = 0; ci < nc && na < k; ++ci) {
                const hyp *src = &alive[s * k + cands[ci].bi];
                const uint32_t tok = cands[ci].tok;
                if (tok == eos || step == max_new) {
                    const int n = src->n + (tok != eos);
                    if (!is_done[s] || mutant == MUT_PUSH_AFTER_DONE) {
                        if (ndone[s] == capdone[s]) {
                            capdone[s] = capdone[s] ? 2 * capdone[s] : 8;
                            dl[s] = realloc(dl[s], (size_t)capdone[s] * sizeof(hyp));
                        }
                        hyp *h = &dl[s][ndone[s]++];
                        h->n = n;
                        h->toks = malloc((size_t)(n ? n : 1) * 4);
                        if (src->n) memcpy(h->toks, src->toks, (size_t)src->n * 4);
                        if (tok != eos) h->toks[src->n] = tok;
                        h->score = cands[ci].score / PEN(mutant == MUT_DONE_LEN ? n : n + 1);
                    }
                    continue;
                }
                hyp *h = &new_alive[na++];
                h->n = src->n + 1;
                h->toks = malloc((size_t)h->n * 4);
                if (src->n) memcpy(h->toks, src->toks, (size_t)src->n * 4);
                h->toks[src->n] = tok;
                h->score = cands[ci].score;
                reorder[nr] = (uint32_t)(s * k + cands[ci].bi);
                next[nr++] = tok;
            }
            float best_done = -INFINITY;
            for (int i = 0; i < ndone[s]; ++i) best_done = fmaxf(best_done, dl[s][i].score);
            const float best_alive =
                na > 0 ? new_alive[0].score / PEN(mutant == MUT_ALIVE_PEN_STEP ? step : step + 1) : -INFINITY;
            const int enough = ndone[s] >= k || mutant == MUT_NO_COUNT;
            if (enough && (mutant == MUT_STOP_STRICT ? best_done > best_alive : best_done >= best_alive)) is_done[s] = 1;
            /* keep the batch rectangular: copies of beam 0 fed EOS, scored -inf */
            while (na < k) {
                reorder[nr] = (uint32_t)(s * k);
                next[nr++] = mutant == MUT_PAD_TOKEN ? 1u : eos;
                new_alive[na].score = mutant == MUT_PAD_SCORE ? 0.f : -INFINITY;
                new_alive[na].n = 0;
                new_alive[na].toks = NULL;
                ++na;
            }
            for (int i = 0; i < nalive[s]; ++i) free(alive[s * k + i].toks);
            for (int i = 0; i < k; ++i) alive[s * k + i] = new_alive[i];
            nalive[s] = k;
        }
        int all = 1;
        for (int s = 0; s < b; ++s) all &= is_done[s];
        if (step == max_new || all) break;
        rc = dec->advance(dec->self, reorder, next, logits);
    }
#undef PEN
    for (int s = 0; s < b; ++s) {
        const hyp *list = ndone[s] ? dl[s] : &alive[s * k];
        const int n = ndone[s] ? ndone[s] : nalive[s];
        int best = -1;
        for (int i = 0; i < n; ++i) { /* Iterator::max_by: the last maximum wins */
            const int32_t ki = total_key(list[i].score), kb = total_key(list[best < 0 ? 0 : best].score);
            const int better = mutant == MUT_FIRST_MAX ? ki > kb : ki >= kb;
            if (best < 0 || better) best = i;
        }
        ntok[s] = 0;
        if (best >= 0) {
            const int nn = list[best].n < max_new ? list[best].n : max_new;
            if (nn) memcpy(out + (size_t)s * max_new, list[best].toks, (size_t)nn * 4);
            ntok[s] = nn;
        }
    }
    for (int s = 0; s < b; ++s) {
        for (int i = 0; i < nalive[s]; ++i) free(alive[s * k + i].toks);
        for (int i = 0; i < ndone[s]; ++i) free(dl[s][i].toks);
        free(dl[s]);
    }
    free(dl); free(ndone); free(capdone); free(alive); free(nalive); free(is_done); free(logits); free(lsm);
    free(vals); free(idx); free(reorder); free(next); free(cands); free(new_alive);
    return rc;
}

/* The model as the beam's decoder: the cache of every row, reordered and fed by the merge. */
typedef struct {
    const orc_model *m;
    orc_state *st;
    uint32_t tgt;
    int rows;
} model_decoder;

static int model_first(void *self, float *out) {
    model_decoder *md = self;
    uint32_t *start = malloc((size_t)md->rows * 2 * 4);
    for (int i = 0; i < md->rows; ++i) {
        start[2 * i] = (uint32_t)md->m->cfg.decoder_start_token_id;
        start[2 * i + 1] = md->tgt;
    }
    const int rc = orc_decode(md->m, md->st, start, 2, out, NULL);
    free(start);
    return rc;
}

static int model_advance(void *self, const uint32_t *reorder, const uint32_t *next, float *out) {
    model_decoder *md = self;
    state_reorder(md->st, reorder, md->rows);
    return orc_decode(md->m, md->st, next, 1, out, NULL);
}

/* src/translator.rs:250-335 */
static int beam_search(const orc_model *m, orc_state *st, int b, uint32_t tgt, int max_new, int k, float lp, int flags,
                       uint32_t *out /* [b][max_new] */, int *ntok) {
    uint32_t *expand = malloc((size_t)b * k * 4);
    for (int i = 0; i < b * k; ++i) expand[i] = (uint32_t)(i / k);
    state_reorder(st, expand, b * k);
    free(expand);
    model_decoder md = {m, st, tgt, b * k};
    const beam_decoder dec = {model_first, model_advance, &md, m->cfg.vocab_size, 1};
    return beam_core(b, k, max_new, lp, (uint32_t)m->cfg.eos_token_id, (flags & ORC_EOS_MASK) != 0, &dec, 0, out,
                     ntok);
}

/* A scripted decoder: each row's history (the tokens fed after [start, tgt], reordered
 * with the row) goes to the caller, which returns that row's log-probabilities. */
typedef struct {
    orc_script_fn fn;
    void *user;
    int rows, len, cap, step;
    uint32_t *hist, *tmp; /* [rows][cap] */
} script_decoder;

static int script_first(void *self, float *out) {
    script_decoder *sd = self;
    sd->step = 1;
    return sd->fn(sd->user, 1, sd->rows, sd->hist, 0, out);
}

static int script_advance(void *self, const uint32_t *reorder, const uint32_t *next, float *out) {
    script_decoder *sd = self;
    if (sd->len + 1 > sd->cap) return -1;
    for (int r = 0; r < sd->rows; ++r) {
        memcpy(sd->tmp + (size_t)r * sd->cap, sd->hist + (size_t)reorder[r] * sd->cap, (size_t)sd->len * 4);
        sd->tmp[(size_t)r * sd->cap + sd->len] = next[r];
    }
    uint32_t *t = sd->hist;
    sd->hist = sd->tmp;
    sd->tmp = t;
    ++sd->len;
    ++sd->step;
    /* rows handed over packed: [rows][len] */
    uint32_t *packed = malloc((size_t)sd->rows * sd->len * 4 + 4);
    for (int r = 0; r < sd->rows; ++r) memcpy(packed + (size_t)r * sd->len, sd->hist + (size_t)r * sd->cap, (size_t)sd->len * 4);
    const int rc = sd->fn(sd->user, sd->step, sd->rows, packed, sd->len, out);
    free(packed);
    return rc;
}

int orc_beam_scripted(int b, int k, int V, uint32_t eos, int max_new, float length_penalty, int flags,
                      orc_script_fn fn, void *user, int mutant, uint32_t *out, int *ntok) {
    if (b <= 0 || k <= 0 || k > V || max_new < 0 || eos >= (uint32_t)V || !fn) return -1;
    script_decoder sd = {fn, user, b * k, 0, max_new + 1, 0, NULL, NULL};
    sd.hist = calloc((size_t)sd.rows * sd.cap, 4);
    sd.tmp = calloc((size_t)sd.rows * sd.cap, 4);
    const beam_decoder dec = {script_first, script_advance, &sd, V, 0};
    const int rc = beam_core(b, k, max_new, length_penalty, eos, (flags & ORC_EOS_MASK) != 0, &dec, mutant, out, ntok);
    free(sd.hist);
    free(sd.tmp);
    return rc;
}

/* src/translator.rs:175-207 for one batch: encode, greedy or beam, truncate each
 * row to its own budget.  out is [b][out_cap]; out_len receives the lengths. */
static int generate_impl(const orc_model *m, const uint32_t *ids, const uint32_t *lens, int b, uint32_t tgt_lang,
                         const orc_gen_options *o, int flags, uint32_t *out, int out_cap, int *out_len,
                         float *min_gap, const uint32_t *sl_ids, int n_sl);

int orc_generate(const orc_model *m, const uint32_t *ids, const uint32_t *lens, int b, uint32_t tgt_lang,
                 const orc_gen_options *o, int flags, uint32_t *out, int out_cap, int *out_len, float *min_gap) {
    return generate_impl(m, ids, lens, b, tgt_lang, o, flags, out, out_cap, out_len, min_gap, NULL, 0);
}

/* Greedy with a shortlist (sl_ids sorted, n_sl > 0): src/translator.rs:184-194 with
 * opts.shortlist, GraphCache::greedy's shortlist branch. */
int orc_generate_sl(const orc_model *m, const uint32_t *ids, const uint32_t *lens, int b, uint32_t tgt_lang,
                    const orc_gen_options *o, int flags, const uint32_t *sl_ids, int n_sl, uint32_t *out, int out_cap,
                    int *out_len, float *min_gap) {
    if (n_sl <= 0 || !sl_ids || o->beam_size > 1) return -1;
    return generate_impl(m, ids, lens, b, tgt_lang, o, flags, out, out_cap, out_len, min_gap, sl_ids, n_sl);
}

static int generate_impl(const orc_model *m, const uint32_t *ids, const uint32_t *lens, int b, uint32_t tgt_lang,
                         const orc_gen_options *o, int flags, uint32_t *out, int out_cap, int *out_len,
                         float *min_gap, const uint32_t *sl_ids, int n_sl) {
    const orc_config *c = &m->cfg;
    if (b <= 0) return 0;
    int max_new = 1;
    for (int i = 0; i < b; ++i) { const int v = budget(c, (int)lens[i], o->max_new_tokens); if (v > max_new) max_new = v; }
    orc_state *st = orc_encode(m, ids, lens, b, max_new, flags, NULL);
    if (!st) return -1;
    uint32_t *toks = calloc((size_t)b * max_new, 4);
    int *nt = calloc((size_t)b, sizeof(int));
    int rc;
    const int sync = o->sync_every > 0 ? o->sync_every : 1;
    uint32_t *off = NULL;
    orc_shortlist sl = {sl_ids, n_sl, ids, NULL};
    if (n_sl > 0) {
        off = malloc((size_t)(b + 1) * 4);
        off[0] = 0;
        for (int i = 0; i < b; ++i) off[i + 1] = off[i] + lens[i];
        sl.off = off;
    }
    if (o->beam_size <= 1) rc = greedy(m, st, b, tgt_lang, max_new, sync, flags, toks, nt, min_gap, n_sl > 0 ? &sl : NULL);
    else rc = beam_search(m, st, b, tgt_lang, max_new, o->beam_size, o->length_penalty, flags, toks, nt);
    for (int i = 0; rc == 0 && i < b; ++i) {
        int n = nt[i];
        const int bud = budget(c, (int)lens[i], o->max_new_tokens);
        if (n > bud) n = bud;
        if (n > out_cap) n = out_cap;
        memcpy(out + (size_t)i * out_cap, toks + (size_t)i * max_new, (size_t)n * 4);
        out_len[i] = n;
    }
    free(toks); free(nt); free(off);
    orc_state_free(st);
    return rc;
}

/* Dequantized-f32 GEMV on raw GGUF rows: y[r][n] = sum_k x[r][k] w[n][k] (f64 accumulation). */
int orc_gemv(uint32_t type, const void *w, int N, int K, const float *x, int rows, float *y) {
    int be, bb;
    if (orc_type_block(type, &be, &bb) || K % be) return -1;
    const size_t row_bytes = (size_t)K / be * bb;
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(| : bad)
    for (int n = 0; n < N; ++n) {
        float *wr = malloc((size_t)K * 4);
        bad |= orc_dequant(type, (const uint8_t *)w + n * row_bytes, K, wr) != 0;
        for (int r = 0; r < rows; ++r) {
            double a = 0;
            for (int k = 0; k < K; ++k) a += (double)x[(size_t)r * K + k] * wr[k];
            y[(size_t)r * N + n] = (float)a;
        }
        free(wr);
    }
    return bad ? -1 : 0;
}
