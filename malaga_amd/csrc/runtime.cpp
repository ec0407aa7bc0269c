#include "runtime.hpp"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <type_traits>

#include "beam.hpp"
#include "gguf.hpp"
#include "quant.hpp"

namespace mlg {

namespace {

constexpr float kLnEps = 1e-5f;          // src/config.rs:58
constexpr size_t kGraphBytes = 32u << 20;  // accounting per captured graph (src/graph.rs:149-150)

std::atomic<long> g_fail_after{-1};

[[noreturn]] void fail(int code, const std::string &msg) { throw Failure{code, msg}; }

uint32_t next_pow2(uint32_t n) {
    uint32_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

template <typename T>
void h2d(T *dst, const std::vector<T> &src, hipStream_t st) {
    if (src.empty()) return;
    check_hip(hipMemcpyAsync(dst, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice, st), "H2D copy");
    check_hip(hipStreamSynchronize(st), "H2D sync");
}

}  // namespace

Staging::~Staging() {
    if (pending_) (void)hipEventSynchronize(ev_);
    if (ev_) (void)hipEventDestroy(ev_);
    if (buf_) (void)hipHostFree(buf_);
}

void Staging::upload(void *dst, const void *src, size_t n, hipStream_t st) {
    if (!n) return;
    const size_t need = (n + 255) & ~size_t(255);
    if (off_ + need > cap_) {
        if (pending_) check_hip(hipEventSynchronize(ev_), "staging wait");
        pending_ = false;
        off_ = 0;
        if (need > cap_) {
            if (buf_) (void)hipHostFree(buf_);
            buf_ = nullptr;
            cap_ = 0;
            void *p = nullptr;
            const size_t cap = std::max(need, size_t(1) << 20);
            check_hip(hipHostMalloc(&p, cap, hipHostMallocDefault), "pinned staging");
            buf_ = static_cast<uint8_t *>(p);
            cap_ = cap;
        }
    }
    if (!ev_) check_hip(hipEventCreateWithFlags(&ev_, hipEventDisableTiming), "event");
    std::memcpy(buf_ + off_, src, n);
    check_hip(hipMemcpyAsync(dst, buf_ + off_, n, hipMemcpyHostToDevice, st), "H2D");
    off_ += need;
    check_hip(hipEventRecord(ev_, st), "event");
    pending_ = true;
}

namespace {

// Device buffers freed at scope exit.
struct DevTemp {
    std::vector<void *> p;
    ~DevTemp() {
        for (auto q : p) dev_free(q);
    }
    template <typename T>
    T *get(size_t n, const char *what) {
        p.push_back(dev_alloc(n * sizeof(T), what));
        return static_cast<T *>(p.back());
    }
};

}  // namespace

void check_hip(hipError_t e, const char *what) {
    if (e == hipSuccess) return;
    if (e == hipErrorOutOfMemory) fail(ERR_OOM, std::string("OUT_OF_MEMORY: ") + what);
    fail(ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

void set_fail_alloc_after(long n) { g_fail_after.store(n); }

void *dev_alloc(size_t bytes, const char *what) {
    const long n = g_fail_after.load();
    if (n >= 0) {  // one-shot test hook
        g_fail_after.store(n - 1);
        if (n == 0) fail(ERR_OOM, std::string("OUT_OF_MEMORY: injected allocation failure (") + what + ")");
    }
    void *p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        fail(ERR_OOM, std::string("OUT_OF_MEMORY: allocating ") + std::to_string(bytes) + " bytes for " + what);
    }
    check_hip(e, what);
    return p;
}

void dev_free(void *p) {
    if (p) (void)hipFree(p);
}

int bucket(int n, int min, int max) {
    return std::max(std::min(int(next_pow2(uint32_t(std::max(n, min)))), max), n);
}

int budget(const ModelConfig &c, int len, int max_new_tokens) {
    const int cap = std::min(c.max_length, c.max_position_embeddings - 2);
    const int v = max_new_tokens > 0 ? max_new_tokens : 2 * len + 16;
    return std::max(1, std::min(v, cap));
}

// ------------------------------------------------------------------ layout

size_t planes_bytes(uint32_t type, int N, int K) { return size_t(type_bytes(type, K)) * size_t(N); }

bool layout_planes(uint32_t type, int N, int K, const uint8_t *src, uint8_t *out, size_t *off_s, size_t *off_d,
                   size_t *total) {
    TypeInfo ti;
    if (!type_info(type, &ti) || K % ti.block_elems) return false;
    const size_t nblk = size_t(N) * (K / ti.block_elems);
    *total = nblk * ti.block_bytes;
    if (type == GGML_Q6_K) {
        *off_s = nblk * 192;
        *off_d = *off_s + nblk * 16;
        for (int64_t i = 0; i < int64_t(nblk); ++i) {
            const uint8_t *b = src + i * 210;
            std::memcpy(out + i * 192, b, 192);
            std::memcpy(out + *off_s + i * 16, b + 192, 16);
            std::memcpy(out + *off_d + i * 2, b + 208, 2);
        }
    } else if (type == GGML_Q8_0) {
        *off_s = nblk * 32;
        *off_d = nblk * 32;
        for (int64_t i = 0; i < int64_t(nblk); ++i) {
            const uint8_t *b = src + i * 34;
            std::memcpy(out + i * 32, b + 2, 32);
            std::memcpy(out + *off_d + i * 2, b, 2);
        }
    } else {
        std::memcpy(out, src, *total);
        *off_s = *off_d = *total;
    }
    return true;
}

size_t lane_major_bytes(uint32_t type, int N, int K) {
    return type == GGML_Q6_K && K % 256 == 0 ? size_t(N) * (K / 256) * 192 : 0;
}

void layout_lane_major(int N, int K, const uint8_t *q_plane, uint8_t *out) {
    const int nb = K / 256, nch = 4 * nb;
    const size_t P = size_t(N) * nb * 64;
    for (int64_t r = 0; r < N; ++r)
        for (int c = 0; c < nch; ++c) {
            // the pieces load_chunk<GGML_Q6_K> reads for chunk c (gemv_core.hpp)
            const uint8_t *qp = q_plane + (size_t(r) * nb + (c >> 2)) * 192;
            const int h2 = (c >> 1) & 1, i = c & 1;
            const size_t o = (size_t(r) * nch + c) * 16;
            std::memcpy(out + o, qp + 64 * h2 + 16 * i, 16);
            std::memcpy(out + P + o, qp + 64 * h2 + 32 + 16 * i, 16);
            std::memcpy(out + 2 * P + o, qp + 128 + 32 * h2 + 16 * i, 16);
        }
}

size_t tile_major_bytes(uint32_t type, int N, int K) {
    const int B = type == GGML_Q6_K ? kQ6TileBytes : type == GGML_Q4_K ? kQ4TileBytes : 0;
    return B && K % 256 == 0 ? size_t((N + 15) / 16) * (K / 256) * B : 0;
}

void layout_tile_major(uint32_t type, int N, int K, const uint8_t *planes, size_t off_s, size_t off_d,
                       uint8_t *out) {
    const int nb = K / 256;
    std::memset(out, 0, tile_major_bytes(type, N, K));
    if (type == GGML_Q4_K) {  // GGUF blocks as they are: header[16] | qs[128]
        for (int t = 0; t < (N + 15) / 16; ++t)
            for (int kb = 0; kb < nb; ++kb) {
                uint8_t *tb = out + (size_t(t) * nb + kb) * kQ4TileBytes;
                for (int r = 0; r < 16 && 16 * t + r < N; ++r) {  // rows past N stay zero
                    const uint8_t *blk = planes + (size_t(16 * t + r) * nb + kb) * 144;
                    std::memcpy(tb + 16 * r, blk, 16);
                    for (int kq = 0; kq < 4; ++kq)
                        for (int g = 0; g < 4; ++g)  // the 8-byte groups MW<GGML_Q4_K>::load reads
                            std::memcpy(tb + 256 + 1024 * (g >> 1) + 16 * (16 * kq + r) + 8 * (g & 1),
                                        blk + 16 + 32 * g + 8 * kq, 8);
                }
            }
        return;
    }
    for (int t = 0; t < (N + 15) / 16; ++t)
        for (int kb = 0; kb < nb; ++kb) {
            uint8_t *tb = out + (size_t(t) * nb + kb) * kQ6TileBytes;
            for (int r = 0; r < 16 && 16 * t + r < N; ++r) {  // rows past N stay zero
                const size_t blk = size_t(16 * t + r) * nb + kb;
                const uint8_t *qp = planes + blk * 192;  // ql[128] | qh[64]
                for (int kq = 0; kq < 4; ++kq) {
                    const int l = 16 * kq + r;
                    for (int nh = 0; nh < 4; ++nh) {  // the dwords MW<GGML_Q6_K>::load reads
                        const int n = nh >> 1, h = nh & 1;
                        std::memcpy(tb + 16 * l + 4 * nh, qp + 64 * n + 16 * h + 4 * kq, 4);
                        std::memcpy(tb + 1024 + 16 * l + 4 * nh, qp + 64 * n + 32 + 16 * h + 4 * kq, 4);
                        std::memcpy(tb + 2048 + 16 * l + 4 * nh, qp + 128 + 32 * n + 16 * h + 4 * kq, 4);
                    }
                }
                std::memcpy(tb + 3072 + 16 * r, planes + off_s + blk * 16, 16);
                std::memcpy(tb + 3328 + 2 * r, planes + off_d + blk * 2, 2);
            }
        }
}

float *Context::gemm_workspace() {
    if (!gemm_ws) gemm_ws = static_cast<float *>(dev_alloc(kGemmWorkspaceBytes, "GEMM workspace"));
    return gemm_ws;
}

Context::~Context() { dev_free(gemm_ws); }

// ------------------------------------------------------------------- model

Batch::~Batch() { dev_free(block); }

StaticState::~StaticState() {
    for (auto p : owned) dev_free(p);
}

Model::~Model() {
    graphs.clear();
    for (auto p : owned_) dev_free(p);
    dev_free(enc_ws_);
}

float *Model::upload_f32(GgufFile &g, const std::string &name, int64_t n) {
    const GgufTensorInfo *t = g.tensor(name);
    if (!t) fail(ERR_FORMAT, "missing tensor " + name);
    if (t->numel() != n) fail(ERR_FORMAT, "tensor " + name + " has " + std::to_string(t->numel()) + " values");
    std::vector<float> host(static_cast<size_t>(n));
    if (!dequantize(t->type, g.tensor_data(*t), n, host.data()))
        fail(ERR_UNSUPPORTED, "tensor " + name + ": unsupported type " + std::to_string(t->type));
    float *d = static_cast<float *>(dev_alloc(size_t(n) * 4, name.c_str()));
    owned_.push_back(d);
    check_hip(hipMemcpy(d, host.data(), size_t(n) * 4, hipMemcpyHostToDevice), "upload");
    weight_bytes += size_t(n) * 4;
    return d;
}

namespace {
const GgufTensorInfo *matrix_info(GgufFile &g, const std::string &name, int n, int k) {
    const GgufTensorInfo *t = g.tensor(name);
    if (!t) fail(ERR_FORMAT, "missing tensor " + name);
    if (t->ne.size() != 2 || int64_t(t->ne[0]) != k || int64_t(t->ne[1]) != n)
        fail(ERR_FORMAT, "tensor " + name + " has an unexpected shape");
    TypeInfo ti;
    if (!type_info(t->type, &ti) || t->type == GGML_BF16)
        fail(ERR_UNSUPPORTED, "tensor " + name + ": unsupported type " + std::to_string(t->type));
    if (k % ti.block_elems) fail(ERR_FORMAT, "tensor " + name + ": row length not a whole number of blocks");
    return t;
}
}  // namespace

DevMatrix Model::upload_matrix(GgufFile &g, const std::string &name, int n, int k, bool head) {
    const GgufTensorInfo *t = matrix_info(g, name, n, k);
    DevMatrix m;
    m.type = t->type;
    m.N = n;
    m.K = k;
    size_t off_s, off_d, total;
    std::vector<uint8_t> host(planes_bytes(t->type, n, k));
    if (!layout_planes(t->type, n, k, g.tensor_data(*t), host.data(), &off_s, &off_d, &total))
        fail(ERR_FORMAT, "tensor " + name + ": row length not a whole number of blocks");
    uint8_t *d = static_cast<uint8_t *>(dev_alloc(total, name.c_str()));
    owned_.push_back(d);
    check_hip(hipMemcpy(d, host.data(), total, hipMemcpyHostToDevice), "upload");
    m.q = d;
    m.s = d + off_s;
    m.d = d + off_d;
    m.bytes = total;
    weight_bytes += total;
    if (head) upload_lane_major(m, host.data());
    upload_tile_major(m, host.data(), off_s, off_d);
    return m;
}

void Model::upload_tile_major(DevMatrix &m, const uint8_t *planes, size_t off_s, size_t off_d) {
    const size_t tb = tile_major_bytes(m.type, m.N, m.K);
    if (!tb) return;
    std::vector<uint8_t> tmh(tb);
    layout_tile_major(m.type, m.N, m.K, planes, off_s, off_d, tmh.data());
    m.tm = static_cast<uint8_t *>(dev_alloc(tb, "matrix (tile-major)"));
    owned_.push_back(m.tm);
    check_hip(hipMemcpy(m.tm, tmh.data(), tb, hipMemcpyHostToDevice), "upload");
    weight_bytes += tb;
}

void Model::upload_lane_major(DevMatrix &m, const uint8_t *q_plane) {
    const size_t lb = lane_major_bytes(m.type, m.N, m.K);
    if (!lb) return;
    std::vector<uint8_t> lm(lb);
    layout_lane_major(m.N, m.K, q_plane, lm.data());
    m.lm = static_cast<uint8_t *>(dev_alloc(lb, "LM head (lane-major quants)"));
    owned_.push_back(m.lm);
    check_hip(hipMemcpy(m.lm, lm.data(), lb, hipMemcpyHostToDevice), "upload");
    weight_bytes += lb;
}

Linear Model::load_linear(GgufFile &g, const std::string &name, int n, int k) {
    Linear l;
    l.w = upload_matrix(g, name + ".weight", n, k);
    l.b = upload_f32(g, name + ".bias", n);
    return l;
}

// dec.blk.{i}{suffix} for i < layers, rows stacked layer after layer (same GGUF type)
Linear Model::load_stacked(GgufFile &g, const std::string &suffix, int layers, int n, int k) {
    Linear l;
    if (layers <= 0) return l;
    std::vector<uint8_t> rows;
    std::vector<float> bias(size_t(layers) * n);
    uint32_t type = 0;
    for (int i = 0; i < layers; ++i) {
        const std::string p = "dec.blk." + std::to_string(i) + suffix;
        const GgufTensorInfo *t = matrix_info(g, p + ".weight", n, k);
        if (i == 0) type = t->type;
        if (t->type != type) fail(ERR_FORMAT, p + ".weight: type differs from layer 0");
        const size_t rb = size_t(type_bytes(type, int64_t(n) * k));
        rows.insert(rows.end(), g.tensor_data(*t), g.tensor_data(*t) + rb);
        const GgufTensorInfo *b = g.tensor(p + ".bias");
        if (!b) fail(ERR_FORMAT, "missing tensor " + p + ".bias");
        if (b->numel() != n || !dequantize(b->type, g.tensor_data(*b), n, bias.data() + size_t(i) * n))
            fail(ERR_FORMAT, "tensor " + p + ".bias: bad shape or type");
    }
    const int N = layers * n;
    std::vector<uint8_t> host(planes_bytes(type, N, k));
    size_t off_s, off_d, total;
    if (!layout_planes(type, N, k, rows.data(), host.data(), &off_s, &off_d, &total))
        fail(ERR_FORMAT, "dec.blk.*" + suffix + ": row length not a whole number of blocks");
    uint8_t *d = static_cast<uint8_t *>(dev_alloc(total, ("dec.blk.*" + suffix).c_str()));
    owned_.push_back(d);
    check_hip(hipMemcpy(d, host.data(), total, hipMemcpyHostToDevice), "upload");
    l.w.type = type;
    l.w.N = N;
    l.w.K = k;
    l.w.q = d;
    l.w.s = d + off_s;
    l.w.d = d + off_d;
    l.w.bytes = total;
    upload_tile_major(l.w, host.data(), off_s, off_d);
    l.b = static_cast<float *>(dev_alloc(bias.size() * 4, ("dec.blk.*" + suffix + " bias").c_str()));
    owned_.push_back(l.b);
    check_hip(hipMemcpy(l.b, bias.data(), bias.size() * 4, hipMemcpyHostToDevice), "upload");
    weight_bytes += total + bias.size() * 4;
    return l;
}

DevMatrix rows_view(const DevMatrix &w, int r0, int n) {
    TypeInfo ti;
    type_info(w.type, &ti);
    const size_t nb = size_t(w.K / ti.block_elems), b0 = size_t(r0) * nb;
    DevMatrix v = w;
    v.N = n;
    v.lm = nullptr;
    v.bytes = size_t(n) * nb * ti.block_bytes;
    // the tile-major copy from tile r0 / 16 on (a view starting inside a tile has none)
    const size_t tb = tile_major_bytes(w.type, 16, w.K);
    v.tm = w.tm && r0 % 16 == 0 ? w.tm + size_t(r0 / 16) * tb : nullptr;
    if (w.type == GGML_Q6_K) {  // planes: quants 192, scales 16, d 2 bytes per block
        v.q = w.q + b0 * 192;
        v.s = w.s + b0 * 16;
        v.d = w.d + b0 * 2;
    } else if (w.type == GGML_Q8_0) {  // quants 32, d 2 bytes per block
        v.q = w.q + b0 * 32;
        v.s = v.d = w.d + b0 * 2;
    } else {
        v.q = w.q + b0 * ti.block_bytes;
        v.s = v.d = v.q + v.bytes;
    }
    return v;
}

LNorm Model::load_ln(GgufFile &g, const std::string &name, int d) {
    LNorm l;
    l.g = upload_f32(g, name + ".weight", d);
    l.b = upload_f32(g, name + ".bias", d);
    return l;
}

// src/config.rs:93-116 and src/model.rs:343-433
void Model::load(const std::string &path) {
    GgufFile g;
    const std::string err = g.open(path);
    if (!err.empty()) fail(ERR_IO, err);
    const GgufValue *arch = g.get("general.architecture");
    if (!arch || arch->type != GV_STRING || arch->s != "nllb")
        fail(ERR_FORMAT, "unsupported architecture, expected 'nllb'");
    auto u = [&](const char *key) -> int {
        const GgufValue *v = g.get(key);
        if (!v || !v->is_int()) fail(ERR_FORMAT, std::string("missing GGUF metadata key '") + key + "'");
        return int(v->u);
    };
    cfg.vocab_size = u("nllb.vocab_size");
    cfg.d_model = u("nllb.embedding_length");
    cfg.encoder_layers = u("nllb.encoder.block_count");
    cfg.decoder_layers = u("nllb.decoder.block_count");
    cfg.encoder_heads = u("nllb.encoder.attention.head_count");
    cfg.decoder_heads = u("nllb.decoder.attention.head_count");
    cfg.encoder_ffn = u("nllb.encoder.feed_forward_length");
    cfg.decoder_ffn = u("nllb.decoder.feed_forward_length");
    cfg.max_position_embeddings = u("nllb.context_length");
    cfg.scale_embedding = u("nllb.scale_embedding");
    cfg.max_length = u("nllb.max_length");
    cfg.bos_token_id = u("tokenizer.ggml.bos_token_id");
    cfg.pad_token_id = u("tokenizer.ggml.padding_token_id");
    cfg.eos_token_id = u("tokenizer.ggml.eos_token_id");
    cfg.decoder_start_token_id = u("tokenizer.ggml.decoder_start_token_id");
    const char *nf = std::getenv("MALAGA_NO_FUSED_STEP");
    no_fuse_ = nf && *nf && std::string(nf) != "0";
    const char *sc = std::getenv("MALAGA_SPLIT_CROSS_STEP");
    split_cross_ = sc && *sc && std::string(sc) != "0";
    const char *sk = std::getenv("MALAGA_SPLIT_K_STEP");
    split_k_step_ = sk && *sk && std::string(sk) != "0";
    const int d = cfg.d_model;
    if (d <= 0 || d % cfg.decoder_heads || d % cfg.encoder_heads || d > 4096 || d % 16)
        fail(ERR_UNSUPPORTED, "unsupported d_model " + std::to_string(d));
    if ((d / cfg.decoder_heads) % 8 || (d / cfg.encoder_heads) % 8)
        fail(ERR_UNSUPPORTED, "head dimension must be a multiple of 8");
    if (!attn_head_size_supported(d / cfg.decoder_heads))
        fail(ERR_UNSUPPORTED, "decoder head size " + std::to_string(d / cfg.decoder_heads) +
                                  " (supported: 8, 16, 32, 64, 128, 256)");

    // src/model.rs:416-420: MALAGA_LAZY_EMBEDDINGS (set, any value) defers the full table
    // when the file has a shortlist
    bool has_sl = false;
    for (const auto &kv : g.metadata()) has_sl |= kv.first.compare(0, 15, "nllb.shortlist.") == 0;
    if (has_sl && std::getenv("MALAGA_LAZY_EMBEDDINGS")) {
        const GgufTensorInfo *t = matrix_info(g, "token_embd.weight", cfg.vocab_size, d);
        embed.type = t->type;
        embed.N = cfg.vocab_size;
        embed.K = d;
        embed.bytes = planes_bytes(t->type, cfg.vocab_size, d);
        embed_host_.assign(g.tensor_data(*t), g.tensor_data(*t) + embed.bytes);
    } else {
        embed = upload_matrix(g, "token_embd.weight", cfg.vocab_size, d, true);
    }
    // src/model.rs:324-340: [sin | cos] in f64, row pad zeroed
    n_pos = cfg.max_position_embeddings + cfg.pad_token_id + 1;
    std::vector<float> table(static_cast<size_t>(n_pos) * d, 0.f);
    const int half = d / 2;
    const double step = std::log(10000.0) / (double(half) - 1.0);
    for (int p = 0; p < n_pos; ++p) {
        if (p == cfg.pad_token_id) continue;
        for (int i = 0; i < half; ++i) {
            const double a = double(p) * std::exp(-double(i) * step);
            table[size_t(p) * d + i] = float(std::sin(a));
            table[size_t(p) * d + half + i] = float(std::cos(a));
        }
    }
    pos = static_cast<float *>(dev_alloc(table.size() * 4, "position table"));
    owned_.push_back(pos);
    check_hip(hipMemcpy(pos, table.data(), table.size() * 4, hipMemcpyHostToDevice), "upload");
    embed_scale = cfg.scale_embedding ? float(std::sqrt(double(d))) : 1.f;

    for (int i = 0; i < cfg.encoder_layers; ++i) {
        const std::string p = "enc.blk." + std::to_string(i);
        EncLayer l;
        l.attn_norm = load_ln(g, p + ".attn_norm", d);
        l.qkv = load_linear(g, p + ".attn_qkv", 3 * d, d);
        l.out = load_linear(g, p + ".attn_out", d, d);
        l.ffn_norm = load_ln(g, p + ".ffn_norm", d);
        l.up = load_linear(g, p + ".ffn_up", cfg.encoder_ffn, d);
        l.down = load_linear(g, p + ".ffn_down", d, cfg.encoder_ffn);
        enc.push_back(l);
    }
    for (int i = 0; i < cfg.decoder_layers; ++i) {
        const std::string p = "dec.blk." + std::to_string(i);
        DecLayer l;
        l.attn_norm = load_ln(g, p + ".attn_norm", d);
        l.qkv = load_linear(g, p + ".attn_qkv", 3 * d, d);
        l.out = load_linear(g, p + ".attn_out", d, d);
        l.cross_norm = load_ln(g, p + ".cross_attn_norm", d);
        l.cross_q = load_linear(g, p + ".cross_attn_q", d, d);
        l.cross_out = load_linear(g, p + ".cross_attn_out", d, d);
        l.ffn_norm = load_ln(g, p + ".ffn_norm", d);
        l.up = load_linear(g, p + ".ffn_up", cfg.decoder_ffn, d);
        l.down = load_linear(g, p + ".ffn_down", d, cfg.decoder_ffn);
        dec.push_back(l);
    }
    cross_kv = load_stacked(g, ".cross_attn_kv", cfg.decoder_layers, 2 * d, d);
    enc_norm = load_ln(g, "enc.output_norm", d);
    dec_norm = load_ln(g, "dec.output_norm", d);
    // src/model.rs:403-412: nllb.shortlist.{code} = ids, lm_head.{code}.weight = their rows
    const std::string prefix = "nllb.shortlist.";
    for (const auto &kv : g.metadata()) {
        if (kv.first.compare(0, prefix.size(), prefix) != 0) continue;
        auto sl = std::make_unique<Shortlist>();
        sl->code = kv.first.substr(prefix.size());
        if (kv.second.type != GV_ARRAY || kv.second.arr.empty())
            fail(ERR_FORMAT, "shortlist " + sl->code + ": expected a non-empty id array");
        for (const GgufValue &v : kv.second.arr) {
            if (!v.is_int() || v.u >= uint64_t(cfg.vocab_size))
                fail(ERR_FORMAT, "shortlist " + sl->code + ": id out of range");
            sl->ids.push_back(uint32_t(v.u));
        }
        // Shortlist::row is a binary search (src/model.rs:246-249): the ids must be sorted
        if (!std::is_sorted(sl->ids.begin(), sl->ids.end()))
            fail(ERR_FORMAT, "shortlist " + sl->code + ": ids not sorted");
        const int n = int(sl->ids.size());
        sl->head = upload_matrix(g, "lm_head." + sl->code + ".weight", n, d, true);
        sl->d_ids = static_cast<uint32_t *>(dev_alloc(size_t(n) * 4, "shortlist ids"));
        owned_.push_back(sl->d_ids);
        check_hip(hipMemcpy(sl->d_ids, sl->ids.data(), size_t(n) * 4, hipMemcpyHostToDevice), "upload");
        shortlists.push_back(std::move(sl));
    }
    check_hip(hipDeviceSynchronize(), "model upload");
}

void Model::ensure_embed() {
    if (embed.q) return;
    std::vector<uint8_t> host(embed.bytes);
    size_t off_s, off_d, total;
    if (!layout_planes(embed.type, embed.N, embed.K, embed_host_.data(), host.data(), &off_s, &off_d, &total))
        fail(ERR_FORMAT, "token_embd.weight: bad layout");
    // the OOM message carries src/model.rs:282-285's hint
    uint8_t *d = static_cast<uint8_t *>(
        dev_alloc(total, "full-vocabulary LM head (token_embd); free some VRAM or decode to a language with a "
                         "shortlist"));
    owned_.push_back(d);
    check_hip(hipMemcpy(d, host.data(), total, hipMemcpyHostToDevice), "upload");
    embed.q = d;
    embed.s = d + off_s;
    embed.d = d + off_d;
    weight_bytes += total;
    upload_lane_major(embed, host.data());
    upload_tile_major(embed, host.data(), off_s, off_d);
    embed_host_.clear();
    embed_host_.shrink_to_fit();
}

DevMatrix Model::gather_embed(const uint32_t *ids, int n, uint8_t *buf) {
    const size_t rb = size_t(type_bytes(embed.type, embed.K));
    std::vector<uint8_t> rows(rb * size_t(n)), planes(planes_bytes(embed.type, n, embed.K));
    for (int i = 0; i < n; ++i) std::memcpy(rows.data() + rb * i, embed_host_.data() + rb * ids[i], rb);
    DevMatrix m;
    m.type = embed.type;
    m.N = n;
    m.K = embed.K;
    size_t off_s, off_d;
    if (!layout_planes(embed.type, n, embed.K, rows.data(), planes.data(), &off_s, &off_d, &m.bytes))
        fail(ERR_FORMAT, "token_embd.weight: bad layout");
    h2d(buf, planes, ctx->stream);
    m.q = buf;
    m.s = buf + off_s;
    m.d = buf + off_d;
    return m;
}

const Shortlist *Model::shortlist(const std::string &code) const {
    for (const auto &sl : shortlists)
        if (sl->code == code) return sl.get();
    return nullptr;
}

void Model::matmul(const Linear &l, const float *x, int rows, float *y, bool relu, const float *resid) {
    hipStream_t st = ctx->stream;
    if (!resid && rows <= gemv_max_batch(l.w)) {
        check_hip(gemv(l.w, x, l.w.K, rows, y, l.w.N, l.b, relu, st), "gemv");
    } else {
        check_hip(gemm(l.w, x, l.w.K, rows, y, l.w.N, l.b, relu, resid, l.w.N, st, ctx->gemm_workspace(),
                       kGemmWorkspaceBytes),
                  "gemm");
    }
}

// src/model.rs:463-500: right-padded ids, embedding * scale + positions (j + pad + 1),
// encoder layers, enc_norm, then the cross K/V of every decoder layer.
std::unique_ptr<Batch> Model::encode(const std::vector<std::vector<uint32_t>> &src) {
    hipStream_t st = ctx->stream;
    auto out = std::make_unique<Batch>();
    const int b = int(src.size());
    int s = 0;
    for (auto &r : src) s = std::max(s, int(r.size()));
    if (b == 0 || s == 0) fail(ERR_INVALID, "empty batch");
    if (s > cfg.max_position_embeddings) fail(ERR_INVALID, "source longer than the position table");
    const int d = cfg.d_model, H = cfg.encoder_heads, hd = d / H, f = cfg.encoder_ffn;
    const uint32_t pad = uint32_t(cfg.pad_token_id);
    // Every encoder operation but the attention is row-wise, so the encoder runs on the
    // packed tokens only (M rows, sentence i at rows soff[i] ..): src/model.rs:480-500 pads
    // the batch to [b, s] and masks the padding in the attention, which computes the same
    // rows.  The batch keeps the [b][s] ids and the [b][H][s][hd] cross K/V of the padded
    // layout (padding positions zero), which the decode state reads.
    std::vector<uint32_t> ids(size_t(b) * s, pad), pids, pidx, soff, rsent, prow;
    out->b = b;
    out->s = s;
    for (int i = 0; i < b; ++i) {
        // a row without tokens would attend over nothing (NaN in src/model.rs:101-109)
        if (src[i].empty()) fail(ERR_INVALID, "empty source row");
        out->lens.push_back(uint32_t(src[i].size()));
        soff.push_back(uint32_t(pids.size()));
        for (int j = 0; j < int(src[i].size()); ++j) {
            if (src[i][j] >= uint32_t(cfg.vocab_size)) fail(ERR_INVALID, "token id out of range");
            ids[size_t(i) * s + j] = src[i][j];
            pids.push_back(src[i][j]);
            pidx.push_back(uint32_t(j) + pad + 1);
            rsent.push_back(uint32_t(i));
            prow.push_back(uint32_t(i * s + j));
        }
    }
    const int M = int(pids.size());
    if (M == 0) fail(ERR_INVALID, "empty batch");
    // scratch: carved from the model's grow-only encoder workspace (256-byte aligned)
    const size_t n_ids = (size_t(M) * 4 + 255) & ~size_t(255), n_lens = (size_t(b) * 4 + 255) & ~size_t(255);
    const size_t n_act = (size_t(M) * d * 4 + 255) & ~size_t(255);
    const size_t n_qkv = (size_t(M) * std::max(3 * d, f) * 4 + 255) & ~size_t(255);
    // cross K/V of all decoder layers per GEMM while the f32 staging stays <= 128 MB
    // (MALAGA_CROSS_KV_STAGING_MB, a test hook, sets another budget; 0: one layer per GEMM)
    size_t staging = size_t(128) << 20;
    if (const char *e = std::getenv("MALAGA_CROSS_KV_STAGING_MB"))
        staging = size_t(std::strtoull(e, nullptr, 10)) << 20;
    const int L = int(dec.size()), per_layer = int(std::min<size_t>(std::max<size_t>(size_t(L), 1),
                                                    std::max<size_t>(1, staging / (size_t(M) * 2 * d * 4))));
    const size_t n_kv = (size_t(M) * 2 * d * 4 * per_layer + 255) & ~size_t(255);
    // lazy embeddings: the batch's token_embd rows, gathered on the host (src/model.rs:269-273)
    const size_t n_rows = embed.q ? 0 : (planes_bytes(embed.type, M, d) + 255) & ~size_t(255);
    const size_t need = 4 * n_ids + 2 * n_lens + 3 * n_act + n_qkv + n_kv + n_rows;
    if (enc_ws_bytes_ < need) {
        check_hip(hipStreamSynchronize(st), "encode");  // a previous call may still use it
        dev_free(enc_ws_);
        enc_ws_ = nullptr;
        enc_ws_bytes_ = 0;
        enc_ws_ = dev_alloc(need, "encoder workspace");
        enc_ws_bytes_ = need;
    }
    uint8_t *wp = static_cast<uint8_t *>(enc_ws_);
    auto carve = [&](size_t bytes) {
        void *p = wp;
        wp += bytes;
        return p;
    };
    uint32_t *d_ids = static_cast<uint32_t *>(carve(n_ids)), *d_pidx = static_cast<uint32_t *>(carve(n_ids));
    uint32_t *d_rsent = static_cast<uint32_t *>(carve(n_ids)), *d_prow = static_cast<uint32_t *>(carve(n_ids));
    uint32_t *d_lens = static_cast<uint32_t *>(carve(n_lens)), *d_soff = static_cast<uint32_t *>(carve(n_lens));
    float *x = static_cast<float *>(carve(n_act)), *h = static_cast<float *>(carve(n_act));
    float *att = static_cast<float *>(carve(n_act));
    float *qkv = static_cast<float *>(carve(n_qkv));
    float *kv = static_cast<float *>(carve(n_kv));
    Staging &up = ctx->staging;
    up.upload(d_pidx, pidx.data(), pidx.size() * 4, st);
    up.upload(d_rsent, rsent.data(), rsent.size() * 4, st);
    up.upload(d_prow, prow.data(), prow.size() * 4, st);
    up.upload(d_soff, soff.data(), soff.size() * 4, st);
    out->ids = ids;
    up.upload(d_lens, out->lens.data(), out->lens.size() * 4, st);
    if (embed.q) {
        up.upload(d_ids, pids.data(), pids.size() * 4, st);
        check_hip(embed_pos_rows(embed, d_ids, d_pidx, M, pos, embed_scale, x, st), "embed");
    } else {
        const DevMatrix rows = gather_embed(pids.data(), M, static_cast<uint8_t *>(carve(n_rows)));
        std::vector<uint32_t> iota(static_cast<size_t>(M));
        std::iota(iota.begin(), iota.end(), 0u);
        up.upload(d_ids, iota.data(), iota.size() * 4, st);
        check_hip(embed_pos_rows(rows, d_ids, d_pidx, M, pos, embed_scale, x, st), "embed");
    }
    // pre-LN layers; each residual projection also produces the next LayerNorm (in the
    // split-K reduction when the GEMM splits K), the last one enc_norm
    if (!enc.empty()) check_hip(layernorm(x, M, d, enc[0].attn_norm.g, enc[0].attn_norm.b, kLnEps, h, st), "layernorm");
    else check_hip(layernorm(x, M, d, enc_norm.g, enc_norm.b, kLnEps, h, st), "layernorm");
    for (size_t li = 0; li < enc.size(); ++li) {
        const EncLayer &l = enc[li];
        const LNorm &next = li + 1 < enc.size() ? enc[li + 1].attn_norm : enc_norm;
        matmul(l.qkv, h, M, qkv, false, nullptr);
        check_hip(attn_prefill(qkv, M, H, hd, d_soff, d_rsent, d_lens, s, att, st), "attn_prefill");
        check_hip(gemm_residual_ln(l.out.w, att, d, M, l.out.b, x, l.ffn_norm.g, l.ffn_norm.b, kLnEps, h, st,
                                   ctx->gemm_workspace(), kGemmWorkspaceBytes),
                  "gemm_residual_ln");
        matmul(l.up, h, M, qkv, true, nullptr);
        check_hip(gemm_residual_ln(l.down.w, qkv, f, M, l.down.b, x, next.g, next.b, kLnEps, h, st,
                                   ctx->gemm_workspace(), kGemmWorkspaceBytes),
                  "gemm_residual_ln");
    }
    const int Hd = cfg.decoder_heads, hdd = d / Hd;
    const size_t kv_elems = size_t(b) * s * d;
    out->block = dev_alloc(std::max<size_t>(dec.size(), 1) * 2 * kv_elems * 4, "cross K/V");
    float *K0 = static_cast<float *>(out->block);
    if (M < b * s)  // padding positions: zero (never attended, but copied into decode states)
        check_hip(hipMemsetAsync(K0, 0, std::max<size_t>(dec.size(), 1) * 2 * kv_elems * 4, st), "memset");
    for (int i = 0; i < L; ++i) {
        out->ck.push_back(K0 + 2 * size_t(i) * kv_elems);
        out->cv.push_back(K0 + (2 * size_t(i) + 1) * kv_elems);
    }
    for (int l0 = 0; l0 < L; l0 += per_layer) {  // layers [l0, l0 + nl) in one GEMM
        const int nl = std::min(per_layer, L - l0);
        const Linear part{rows_view(cross_kv.w, l0 * 2 * d, nl * 2 * d), cross_kv.b + size_t(l0) * 2 * d};
        matmul(part, h, M, kv, false, nullptr);
        check_hip(split_cross_kv(kv, M, d_prow, s, Hd, hdd, nl, K0 + 2 * size_t(l0) * kv_elems, kv_elems, st),
                  "split_cross_kv");
    }
    // no wait: the batch's users run on the same stream
    check_hip(hipGetLastError(), "encode");
    return out;
}

std::unique_ptr<StaticState> Model::new_state(int b, int s, int m, bool logits, bool row_map, const Shortlist *sl,
                                              bool kv32) {
    auto st = std::make_unique<StaticState>();
    st->b = b;
    st->s = s;
    st->m = m;
    st->sl = sl;
    st->kv32 = kv32;
    const DevMatrix &head = sl ? sl->head : embed;
    const int d = cfg.d_model, H = cfg.decoder_heads, hd = d / H, L = cfg.decoder_layers, V = cfg.vocab_size;
    auto get = [&](size_t bytes, const char *what) {
        void *p = dev_alloc(bytes, what);
        st->owned.push_back(p);
        st->bytes += bytes;
        return p;
    };
    st->ids = static_cast<uint32_t *>(get(size_t(b) * 4, "ids"));
    st->step = static_cast<uint32_t *>(get(4, "step"));
    st->lens = static_cast<uint32_t *>(get(size_t(b) * 4, "lens"));
    st->out = static_cast<uint32_t *>(get(size_t(b) * m * 4, "out"));
    st->outv = static_cast<float *>(get(size_t(b) * m * 4, "winning logits"));
    st->err = static_cast<uint32_t *>(get(4, "non-finite flag"));
    st->finished = static_cast<uint8_t *>(get(size_t(b), "finished"));
    st->row_src = static_cast<uint32_t *>(get(size_t(b) * 4, "source rows"));
    // one block each for the self and the cross K/V of every layer (layer l: K, then V);
    // slots past the step are read (and masked) by the fused attention: keep them finite
    const size_t self_pair = size_t(b) * H * m * hd, cross_pair = size_t(b) * H * s * hd, es = kv32 ? 4 : 2;
    void *self_kv = get(std::max<size_t>(2 * L * self_pair, 1) * es, "self K/V");
    void *cross_kv = get(std::max<size_t>(2 * L * cross_pair, 1) * es, "cross K/V");
    check_hip(hipMemsetAsync(self_kv, 0, 2 * L * self_pair * es, ctx->stream), "memset");
    check_hip(hipMemsetAsync(cross_kv, 0, 2 * L * cross_pair * es, ctx->stream), "memset");
    for (int i = 0; i < L; ++i) {
        if (kv32) {
            st->kc32.push_back(static_cast<float *>(self_kv) + 2 * i * self_pair);
            st->vc32.push_back(static_cast<float *>(self_kv) + (2 * i + 1) * self_pair);
            st->ck32.push_back(static_cast<float *>(cross_kv) + 2 * i * cross_pair);
            st->cv32.push_back(static_cast<float *>(cross_kv) + (2 * i + 1) * cross_pair);
        } else {
            st->kc.push_back(static_cast<__half *>(self_kv) + 2 * i * self_pair);
            st->vc.push_back(static_cast<__half *>(self_kv) + (2 * i + 1) * self_pair);
            st->ck.push_back(static_cast<__half *>(cross_kv) + 2 * i * cross_pair);
            st->cv.push_back(static_cast<__half *>(cross_kv) + (2 * i + 1) * cross_pair);
        }
    }
    // rows padded to 16: the decode-GEMM step keeps x in fragment order (whole row tiles)
    const size_t bp = size_t(b + 15) / 16 * 16;
    st->x = static_cast<float *>(get(bp * d * 4, "x"));
    check_hip(hipMemsetAsync(st->x, 0, bp * d * 4, ctx->stream), "memset");
    st->xb = static_cast<float *>(get(size_t(b) * d * 4, "x (second buffer)"));
    st->qc = static_cast<float *>(get(size_t(b) * d * 4, "cross q"));
    st->fused = !kv32 && fusable(b, m, s) && (!sl || step_embed_supported(dec[0].qkv.w.type, sl->head.type));
    if (st->fused) {
        st->part = static_cast<float *>(get(size_t(H) * b * d * 4, "attention partial sums"));
        st->part2 = static_cast<float *>(get(size_t(H) * b * d * 4, "cross attention partial sums"));
    }
    if (!st->fused && dgemm_step_ok(b))
        st->lnstat = static_cast<double *>(get(size_t(d / 16) * b * 2 * sizeof(double), "LayerNorm statistics"));
    st->h = static_cast<float *>(get(size_t(b) * d * 4, "h"));
    st->y = static_cast<float *>(get(size_t(b) * d * 4, "y"));
    // att and u: rows padded to 16, zero-filled (the decode-GEMM step keeps them as split
    // fragments, whose row tiles are stored whole)
    st->att = static_cast<float *>(get(bp * d * 4, "att"));
    st->q = static_cast<float *>(get(size_t(b) * d * 4, "q"));
    st->qkv = static_cast<float *>(get(size_t(b) * 3 * d * 4, "qkv"));
    st->u = static_cast<float *>(get(bp * cfg.decoder_ffn * 4, "ffn"));
    check_hip(hipMemsetAsync(st->att, 0, bp * d * 4, ctx->stream), "memset");
    check_hip(hipMemsetAsync(st->u, 0, bp * cfg.decoder_ffn * 4, ctx->stream), "memset");
    if (logits || b > gemv_max_batch(head))
        st->logits = static_cast<float *>(get(size_t(b) * (sl ? head.N : V) * 4, "logits"));
    if (sl) {  // src/graph.rs:76-79
        st->src_ids = static_cast<uint32_t *>(get(size_t(b) * s * 4, "source ids"));
        st->src_emb = static_cast<float *>(get(size_t(b) * s * d * 4, "source embeddings"));
        st->sl_row = static_cast<uint32_t *>(get(size_t(b) * 4, "shortlist rows"));
        st->src_row = static_cast<uint32_t *>(get(size_t(b) * 4, "source positions"));
        st->spv = static_cast<float *>(get(size_t(b) * s * 4, "source logits"));
        st->spi = static_cast<uint32_t *>(get(size_t(b) * s * 4, "source logits"));
        if (!embed.q) {
            st->src_q = static_cast<uint8_t *>(get(planes_bytes(embed.type, b * s, d), "source rows"));
            st->src_iota = static_cast<uint32_t *>(get(size_t(b) * s * 4, "source rows"));
            std::vector<uint32_t> iota(size_t(b) * s);
            std::iota(iota.begin(), iota.end(), 0u);
            h2d(st->src_iota, iota, ctx->stream);
        }
    }
    if (row_map) {  // identity until a beam reorder rewrites it
        st->rows = static_cast<uint32_t *>(get(size_t(b) * m * 4, "beam cache rows"));
        std::vector<uint32_t> id(size_t(b) * m);
        for (int r = 0; r < b; ++r)
            for (int j = 0; j < m; ++j) id[size_t(r) * m + j] = uint32_t(r);
        h2d(st->rows, id, ctx->stream);
    }
    st->parts = std::max(gemv_argmax_parts(head, b), 64);
    if (b > gemv_max_batch(head) && gemm_argmax_supported(head, b))
        st->parts = std::max(st->parts, gemm_argmax_parts(head, b));
    st->pv = static_cast<float *>(get(size_t(b) * st->parts * 4, "argmax partials"));
    st->pi = static_cast<uint32_t *>(get(size_t(b) * st->parts * 4, "argmax partials"));
    check_hip(hipStreamSynchronize(ctx->stream), "state");
    return st;
}

// src/graph.rs:91-118: cross K/V and lens of the batch, start token, step 0.
// Row r of the state takes source row row_of[r]; rows past row_of.size() are idle.
void Model::reset_state(StaticState &st, const Batch &src, const std::vector<uint32_t> &row_of, uint32_t start) {
    hipStream_t s = ctx->stream;
    const int H = cfg.decoder_heads, hd = cfg.d_model / H, n = int(row_of.size());
    if (n > st.b) fail(ERR_INVALID, "reset_state: more source rows than state rows");
    uint32_t *d_map = st.row_src;
    Staging &up = ctx->staging;
    up.upload(d_map, row_of.data(), row_of.size() * 4, s);
    // every layer's K and V in one launch: both blocks hold layer l's K, then its V
    // (src/graph.rs:94-97 stores them as f16; the generic path keeps f32)
    const size_t src_pair = size_t(src.b) * src.s * cfg.d_model, dst_pair = size_t(st.b) * H * st.s * hd;
    if (!st.ck.empty())
        check_hip(copy_cross(src.ck[0], src_pair, d_map, n, H, src.s, hd, st.ck[0], dst_pair, st.s,
                             2 * int(st.ck.size()), s),
                  "copy_cross");
    if (!st.ck32.empty())
        check_hip(copy_cross(src.ck[0], src_pair, d_map, n, H, src.s, hd, st.ck32[0], dst_pair, st.s,
                             2 * int(st.ck32.size()), s),
                  "copy_cross");
    std::vector<uint32_t> lens(static_cast<size_t>(st.b), 1u);
    for (int r = 0; r < n; ++r) lens[r] = src.lens[row_of[r]];
    up.upload(st.lens, lens.data(), lens.size() * 4, s);
    check_hip(fill_u32(st.ids, start, size_t(st.b), s), "fill");
    check_hip(fill_u32(st.step, 0, 1, s), "fill");
    check_hip(fill_u32(st.err, 0, 1, s), "fill");
    if (st.sl) {
        // src/graph.rs:98-108: source ids of every row (pad past the row's length, idle
        // rows all pad) and their token_embd rows
        if (src.s > st.s) fail(ERR_INVALID, "reset_state: source longer than the state");
        const uint32_t pad = uint32_t(cfg.pad_token_id);
        std::vector<uint32_t> ids(size_t(st.b) * st.s, pad);
        for (int r = 0; r < n; ++r)
            std::copy_n(src.ids.begin() + size_t(row_of[r]) * src.s, src.s, ids.begin() + size_t(r) * st.s);
        up.upload(st.src_ids, ids.data(), ids.size() * 4, s);
        if (embed.q) {
            check_hip(embed_rows(embed, st.src_ids, st.b * st.s, st.src_emb, s), "embed_rows");
        } else {
            if (!st.src_q) fail(ERR_INVALID, "reset_state: state without source row buffers");
            const DevMatrix rows = gather_embed(ids.data(), st.b * st.s, st.src_q);
            check_hip(embed_rows(rows, st.src_iota, st.b * st.s, st.src_emb, s), "embed_rows");
        }
        set_shortlist_input(st, start);
    }
    std::vector<uint8_t> fin(static_cast<size_t>(st.b));
    for (int r = 0; r < st.b; ++r) fin[r] = r >= n;
    up.upload(st.finished, fin.data(), fin.size(), s);
}

// src/graph.rs:121-130 (set_ids): every row's next input is vocabulary id `id`.
void Model::set_shortlist_input(StaticState &st, uint32_t id) {
    const int row = st.sl->row(id);
    if (row < 0) fail(ERR_INVALID, "token " + std::to_string(id) + " missing from the shortlist");
    check_hip(fill_u32(st.sl_row, uint32_t(row), size_t(st.b), ctx->stream), "fill");
    check_hip(fill_u32(st.src_row, kNoRow, size_t(st.b), ctx->stream), "fill");
}

bool Model::fusable(int b, int m, int s) const {
    if (no_fuse_ || b > 4 || dec.empty()) return false;
    const int d = cfg.d_model, H = cfg.decoder_heads, hd = d / H;
    if (!step_embed_supported(dec[0].qkv.w.type, embed.type)) return false;
    for (const DecLayer &l : dec) {
        for (const Linear *lin : {&l.qkv, &l.cross_q, &l.up, &l.down})
            if (!step_fusable(lin->w, b, d)) return false;
        const int ps = step_head_parts(l.out.w, b, d, H, hd, m), pc = step_head_parts(l.cross_out.w, b, d, H, hd, s);
        if (ps < 1 || ps > H || pc < 1 || pc > H) return false;
    }
    return true;
}

namespace {
// The f16 hi / lo split of the MFMA operands holds |x| < 65520; an activation beyond it
// becomes NaN, and every logit of its row with it.
constexpr const char *kNonFiniteLogits =
    "decoder produced no finite logit for a row (an activation beyond the f16 range of the MFMA operands?)";

// Layer i's self and cross caches in the state's precision: f(kc, vc, ck, cv) with __half
// pointers (the graph step) or float pointers (the generic path).
template <typename F>
void with_kv(const StaticState &st, size_t i, F &&f) {
    if (st.kv32) f(st.kc32[i], st.vc32[i], st.ck32[i], st.cv32[i]);
    else f(st.kc[i], st.vc[i], st.ck[i], st.cv[i]);
}
}  // namespace

// src/model.rs:552-612 as six fused launches per layer (k_step.hip).
float *Model::step_fused(StaticState &st, bool final_ln) {
    hipStream_t s = ctx->stream;
    const int B = st.b, d = cfg.d_model, H = cfg.decoder_heads, hd = d / H;
    float *cur = st.x, *nxt = st.xb;
    for (size_t i = 0; i < dec.size(); ++i) {
        const DecLayer &l = dec[i];
        if (i == 0) {
            // src/model.rs:558-562: with a shortlist the input is a shortlist row or a source token
            const SrcEmb src = st.sl ? SrcEmb{st.src_emb, st.src_row, st.s} : SrcEmb{};
            check_hip(step_qkv(l.qkv.w, l.qkv.b, B, d, st.sl ? &st.sl->head : &embed, st.sl ? st.sl_row : st.ids,
                               pos, uint32_t(cfg.pad_token_id + 1), embed_scale, nullptr, nullptr, cur,
                               l.attn_norm.g, l.attn_norm.b, kLnEps, st.step, st.q, st.kc[i], st.vc[i], H, hd, st.m,
                               s, src),
                      "step_qkv");
        } else {
            check_hip(step_qkv(l.qkv.w, l.qkv.b, B, d, nullptr, st.ids, pos, 0, 1.f, cur, st.y, nxt, l.attn_norm.g,
                               l.attn_norm.b, kLnEps, st.step, st.q, st.kc[i], st.vc[i], H, hd, st.m, s),
                      "step_qkv");
            std::swap(cur, nxt);
        }
        const int ps = step_head_parts(l.out.w, B, d, H, hd, st.m);
        check_hip(step_attn_head(l.out.w, B, d, st.q, st.kc[i], st.vc[i], H, hd, st.m, nullptr, st.step, st.part, s,
                                 st.rows),
                  "step_attn_head");
        const int pc = step_head_parts(l.cross_out.w, B, d, H, hd, st.s);
        const float *cpart = st.part;
        if (!split_cross_ && step_cross_fusable(l.cross_q.w, l.cross_out.w, B, d, H, hd, st.s, ps)) {
            // cross_q + cross attention + out-projection slice in one launch
            check_hip(step_cross_attn(l.cross_q.w, l.cross_q.b, l.cross_out.w, B, d, cur, st.part, ps, l.out.b, nxt,
                                      l.cross_norm.g, l.cross_norm.b, kLnEps, st.ck[i], st.cv[i], H, hd, st.s,
                                      st.lens, st.part2, s),
                      "step_cross_attn");
            cpart = st.part2;
        } else {
            check_hip(step_resid_proj(l.cross_q.w, l.cross_q.b, false, B, d, cur, st.part, ps, l.out.b, nxt,
                                      l.cross_norm.g, l.cross_norm.b, kLnEps, st.qc, s),
                      "step_cross_q");
            check_hip(step_attn_head(l.cross_out.w, B, d, st.qc, st.ck[i], st.cv[i], H, hd, st.s, st.lens, nullptr,
                                     st.part, s),
                      "step_attn_head");
        }
        std::swap(cur, nxt);
        check_hip(step_resid_proj(l.up.w, l.up.b, true, B, d, cur, cpart, pc, l.cross_out.b, nxt, l.ffn_norm.g,
                                  l.ffn_norm.b, kLnEps, st.u, s),
                  "step_up");
        std::swap(cur, nxt);
        check_hip(step_proj(l.down.w, l.down.b, B, st.u, st.y, s), "step_down");
    }
    // h = dec_norm(x + y) for the LM head
    if (final_ln) check_hip(residual_ln(cur, st.y, B, d, dec_norm.g, dec_norm.b, kLnEps, st.h, s), "residual_ln");
    return cur;
}

void Model::lm_head(StaticState &st, bool greedy_mode, int mask_id, const float *ln_x) {
    hipStream_t s = ctx->stream;
    const int B = st.b, d = cfg.d_model;
    if (greedy_mode) {
        // src/model.rs:597-610: the shortlist head (its rows masked by their vocabulary
        // id) or the tied full head
        const DevMatrix &head = st.sl ? st.sl->head : embed;
        const int V = head.N, hmask = st.sl && mask_id >= 0 ? st.sl->row(uint32_t(mask_id)) : mask_id;
        int parts = 64;
        if (B <= gemv_max_batch(head)) {
            const GemvLn ln{ln_x, st.y, dec_norm.g, dec_norm.b, kLnEps, st.h};
            check_hip(gemv_argmax(head, st.h, d, B, hmask, st.pv, st.pi, &parts, s, ln_x ? &ln : nullptr), "lm_head");
        } else if (gemm_argmax_supported(head, B)) {
            check_hip(gemm_argmax(head, st.h, d, B, hmask, st.pv, st.pi, &parts, s), "lm_head");
        } else {
            check_hip(gemm(head, st.h, d, B, st.logits, V, nullptr, false, nullptr, 0, s, ctx->gemm_workspace(),
                           kGemmWorkspaceBytes),
                      "lm_head");
            check_hip(argmax_partial(st.logits, B, V, V, hmask, st.pv, st.pi, parts, s), "argmax");
        }
        SlFinalize sl;
        if (st.sl) {  // the source tokens: logits at candidate indices V + j (kernels/malaga.cu:229-243)
            check_hip(source_logits(st.h, st.src_emb, st.src_ids, B, st.s, d, mask_id, V, st.spv, st.spi, s),
                      "source_logits");
            sl = SlFinalize{st.sl->d_ids, V, st.spv, st.spi, st.src_ids, st.s, st.sl_row, st.src_row};
        }
        check_hip(greedy_finalize(st.pv, st.pi, parts, B, st.finished, st.ids, st.out, st.m, st.step,
                                  uint32_t(cfg.eos_token_id), uint32_t(cfg.pad_token_id), s, sl, st.outv, st.err),
                  "greedy_finalize");
    } else {
        const int V = cfg.vocab_size;
        if (st.sl) fail(ERR_UNSUPPORTED, "shortlist decoding is greedy only");
        if (B <= gemv_max_batch(embed))
            check_hip(gemv(embed, st.h, d, B, st.logits, V, nullptr, false, s), "lm_head");
        else
            check_hip(gemm(embed, st.h, d, B, st.logits, V, nullptr, false, nullptr, 0, s, ctx->gemm_workspace(),
                           kGemmWorkspaceBytes),
                      "lm_head");
        check_hip(inc_u32(st.step, s), "step");
    }
}

void Model::step(StaticState &st, bool greedy_mode, int mask_id) {
    if (st.fused) {
        // greedy batches up to the register GEMV fold the final LayerNorm into the head
        const DevMatrix &head = st.sl ? st.sl->head : embed;
        const bool fold = greedy_mode && st.b <= gemv_max_batch(head) && (head.type == GGML_Q4_K || head.type == GGML_Q5_K || head.type == GGML_Q6_K ||
                                                                      head.type == GGML_Q8_0);
        float *x = step_fused(st, !fold);
        lm_head(st, greedy_mode, mask_id, fold ? x : nullptr);
        return;
    }
    if (st.lnstat) {
        step_dgemm(st, greedy_mode, mask_id);
        return;
    }
    hipStream_t s = ctx->stream;
    const int B = st.b, d = cfg.d_model, H = cfg.decoder_heads, hd = d / H;
    const SrcEmb src = st.sl ? SrcEmb{st.src_emb, st.src_row, st.s} : SrcEmb{};
    check_hip(embed_pos_ln(st.sl ? st.sl->head : embed, st.sl ? st.sl_row : st.ids, B, pos, st.step,
                           uint32_t(cfg.pad_token_id + 1), embed_scale, dec[0].attn_norm.g, dec[0].attn_norm.b,
                           kLnEps, st.x, st.h, s, src),
              "embed_pos_ln");
    // x += y W^T + b; h = LayerNorm(x): register GEMV + residual_ln for small
    // batches, else the MFMA GEMM with the residual and LayerNorm in its reduction
    auto project_residual_ln = [&](const Linear &l, const float *in, const LNorm &n) {
        if (B <= gemv_max_batch(l.w)) {
            matmul(l, in, B, st.y, false, nullptr);
            check_hip(residual_ln(st.x, st.y, B, d, n.g, n.b, kLnEps, st.h, s), "residual_ln");
        } else {
            check_hip(gemm_residual_ln(l.w, in, l.w.K, B, l.b, st.x, n.g, n.b, kLnEps, st.h, s, ctx->gemm_workspace(),
                                       kGemmWorkspaceBytes),
                      "gemm_residual_ln");
        }
    };
    for (size_t i = 0; i < dec.size(); ++i) {
        const DecLayer &l = dec[i];
        with_kv(st, i, [&](auto *kc, auto *vc, auto *ck, auto *cv) {
            if (B <= gemv_max_batch(l.qkv.w)) {
                matmul(l.qkv, st.h, B, st.qkv, false, nullptr);
                check_hip(qkv_split(st.qkv, B, H, hd, st.m, st.step, st.q, kc, vc, s), "qkv_split");
            } else {
                check_hip(gemm_qkv(l.qkv.w, st.h, d, B, l.qkv.b, H, hd, st.m, st.step, st.q, kc, vc, st.qkv, s,
                                   ctx->gemm_workspace(), kGemmWorkspaceBytes),
                          "gemm_qkv");
            }
            check_hip(attn_decode(st.q, kc, vc, B, H, hd, st.m, nullptr, st.step, st.att, s, st.rows), "attn");
            project_residual_ln(l.out, st.att, l.cross_norm);
            matmul(l.cross_q, st.h, B, st.q, false, nullptr);
            check_hip(attn_decode(st.q, ck, cv, B, H, hd, st.s, st.lens, nullptr, st.att, s), "attn");
        });
        project_residual_ln(l.cross_out, st.att, l.ffn_norm);
        matmul(l.up, st.h, B, st.u, true, nullptr);
        project_residual_ln(l.down, st.u, i + 1 < dec.size() ? dec[i + 1].attn_norm : dec_norm);
    }
    // st.h is dec_norm(x): tied LM head
    lm_head(st, greedy_mode, mask_id);
}

bool Model::dgemm_step_ok(int b) const {
    // LayerNorm and QKV projections take K = d_model in one K block per wave: d <= 2048
    if (split_k_step_ || dec.empty() || b > kDgemmMaxRows || cfg.d_model % 16 || cfg.d_model > 2048) return false;
    for (const DecLayer &l : dec) {
        if (b <= gemv_max_batch(l.qkv.w)) return false;  // the register GEMVs serve small batches
        for (const Linear *lin : {&l.qkv, &l.out, &l.cross_q, &l.cross_out, &l.up, &l.down})
            if (!dgemm_supported(lin->w, b)) return false;
    }
    return true;
}

// src/model.rs:552-612 for batches of 5..64 rows: eight launches per layer, six decode
// GEMMs (k_dgemm.hip) and the two attentions.  The LayerNorms live in the GEMMs: each
// projection that adds to the residual stream x also leaves the new rows' statistics in
// st.lnstat, and the next projection that takes LayerNorm(x) normalizes x as it loads it.
void Model::step_dgemm(StaticState &st, bool greedy_mode, int mask_id) {
    hipStream_t s = ctx->stream;
    const int B = st.b, d = cfg.d_model, H = cfg.decoder_heads, hd = d / H, f = cfg.decoder_ffn;
    const SrcEmb src = st.sl ? SrcEmb{st.src_emb, st.src_row, st.s} : SrcEmb{};
    // x = embedding + position (fragment order), h = LayerNorm(x) with layer 0's attn_norm
    check_hip(embed_pos_ln(st.sl ? st.sl->head : embed, st.sl ? st.sl_row : st.ids, B, pos, st.step,
                           uint32_t(cfg.pad_token_id + 1), embed_scale, dec[0].attn_norm.g, dec[0].attn_norm.b,
                           kLnEps, st.x, st.h, s, src, true),
              "embed_pos_ln");
    auto ln = [&](const LNorm &n) { return DgemmLn{st.lnstat, n.g, n.b, kLnEps}; };
    for (size_t i = 0; i < dec.size(); ++i) {
        const DecLayer &l = dec[i];
        const DgemmLn ln_attn = ln(l.attn_norm), ln_cross = ln(l.cross_norm), ln_ffn = ln(l.ffn_norm);
        with_kv(st, i, [&](auto *kc, auto *vc, auto *ck, auto *cv) {
            check_hip(dgemm_qkv(l.qkv.w, i == 0 ? st.h : st.x, d, B, i == 0 ? nullptr : &ln_attn, l.qkv.b, H, hd,
                                st.m, st.step, st.q, kc, vc, s),
                      "dgemm_qkv");
            // x in fragment order, att and u as split f16 hi / lo fragments: the A-operand
            // order of the decode GEMMs (frag_index, device.hpp)
            check_hip(attn_decode(st.q, kc, vc, B, H, hd, st.m, nullptr, st.step, st.att, s, st.rows, true), "attn");
            check_hip(dgemm_resid(l.out.w, st.att, d, B, l.out.b, st.x, st.lnstat, s, true), "dgemm_out");
            const bool fused_cross = !split_cross_ && dgemm_cross_attn_supported(l.cross_q.w, B, H, hd);
            if (fused_cross) {
                check_hip(dgemm_cross_attn(l.cross_q.w, st.x, B, ln_cross, l.cross_q.b, ck, cv, H, hd, st.s, st.lens,
                                           st.att, s),
                          "dgemm_cross_attn");
            } else {
                // where the one-launch cross attention exists, its q is k_dgemm's bit for bit:
                // the two-launch form keeps k_dgemm too, so that both give the same logits
                check_hip(dgemm_store(l.cross_q.w, st.x, d, B, &ln_cross, l.cross_q.b, false, st.q, d, s, false,
                                      !dgemm_cross_attn_supported(l.cross_q.w, B, H, hd)),
                          "dgemm_cross_q");
                check_hip(attn_decode(st.q, ck, cv, B, H, hd, st.s, st.lens, nullptr, st.att, s, nullptr, true),
                          "attn");
            }
        });
        check_hip(dgemm_resid(l.cross_out.w, st.att, d, B, l.cross_out.b, st.x, st.lnstat, s, true), "dgemm_cross_out");
        check_hip(dgemm_store(l.up.w, st.x, d, B, &ln_ffn, l.up.b, true, st.u, f, s, true), "dgemm_up");
        check_hip(dgemm_resid(l.down.w, st.u, f, B, l.down.b, st.x, st.lnstat, s, true), "dgemm_down");
    }
    // st.h = dec_norm(x): tied LM head
    check_hip(layernorm_frag(st.x, B, d, dec_norm.g, dec_norm.b, kLnEps, st.h, s), "layernorm");
    lm_head(st, greedy_mode, mask_id);
}

// ------------------------------------------------------------ graph cache

namespace {
// Rust's str::parse::<usize>: the whole string is decimal digits (an optional leading
// '+'), else no value.
bool parse_usize(const char *s, size_t *out) {
    if (!s) return false;
    if (*s == '+') ++s;
    if (!*s) return false;
    size_t v = 0;
    for (; *s; ++s) {
        if (*s < '0' || *s > '9') return false;
        const size_t digit = size_t(*s - '0');
        if (v > (SIZE_MAX - digit) / 10) return false;  // overflows usize: a parse error
        v = v * 10 + digit;
    }
    *out = v;
    return true;
}

// src/graph.rs:184: capture stays on when the variable is unset, empty or "0"
bool graph_switch_on(const char *name) {
    const char *v = std::getenv(name);
    return !v || !*v || std::string(v) == "0";
}
}  // namespace

// src/graph.rs:182-186.  MALAGA_NO_HIP_GRAPH is this backend's name for the reference's
// MALAGA_NO_CUDA_GRAPH; either turns capture off.
GraphCache::GraphCache(Model *m) : model_(m) {
    size_t mb = 512;
    if (!parse_usize(std::getenv("MALAGA_GRAPH_CACHE_MB"), &mb)) mb = 512;
    max_bytes_ = mb << 20;  // graph.rs:185 (the shift drops high bits, as Rust's << does)
    capture_ = graph_switch_on("MALAGA_NO_CUDA_GRAPH") && graph_switch_on("MALAGA_NO_HIP_GRAPH");
}

GraphCache::~GraphCache() {
    clear();
    if (fin_host_) (void)hipHostFree(fin_host_);
    if (fin_ev_) (void)hipEventDestroy(fin_ev_);
}

size_t GraphCache::Entry::bytes() const { return st->bytes + (exec ? kGraphBytes : 0); }

size_t GraphCache::graphs() const {
    size_t n = 0;
    for (auto &e : entries_) n += e.exec != nullptr;
    return n;
}

// src/graph.rs:193-200, 325-335: destroyed graphs' memory goes back to the driver
void GraphCache::clear() {
    bool had_graphs = false;
    for (auto &e : entries_)
        if (e.exec) {
            (void)hipGraphExecDestroy(e.exec);
            had_graphs = true;
        }
    entries_.clear();
    if (had_graphs) trim_graph_memory();
}

void GraphCache::trim_graph_memory() {
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGraphMemTrim(dev);
}

// src/graph.rs:301-323: drop least recently used entries (never `keep`) while the
// entries plus one graph's reserve exceed the budget
void GraphCache::evict(const Entry *keep) {
    bool dropped_graph = false;
    for (;;) {
        size_t total = kGraphBytes;
        for (auto &e : entries_) total += e.bytes();
        if (total <= max_bytes_ || entries_.size() <= 1) break;
        auto victim = entries_.end();
        for (auto it = entries_.begin(); it != entries_.end(); ++it)
            if (&*it != keep && (victim == entries_.end() || it->last_used < victim->last_used)) victim = it;
        if (victim == entries_.end()) break;
        if (victim->exec) {
            (void)hipGraphExecDestroy(victim->exec);
            dropped_graph = true;
        }
        entries_.erase(victim);
    }
    if (dropped_graph) trim_graph_memory();
}

std::vector<GraphCache::Key> GraphCache::keys() const {
    std::vector<const Entry *> order;
    for (auto &e : entries_) order.push_back(&e);
    std::stable_sort(order.begin(), order.end(),
                     [](const Entry *a, const Entry *b) { return a->last_used < b->last_used; });
    std::vector<Key> out;
    for (const Entry *e : order) out.push_back(Key{e->b, e->s, e->m, e->exec != nullptr});
    return out;
}

std::vector<std::vector<uint32_t>> GraphCache::greedy(const Batch &src, uint32_t tgt_lang, int max_new,
                                                      int sync_every, bool eos_mask, bool use_graph,
                                                      const Shortlist *sl, std::vector<std::vector<float>> *top) {
    try {
        return run(src, tgt_lang, max_new, sync_every, eos_mask, use_graph, sl, top);
    } catch (const Failure &f) {
        // src/graph.rs:214-222: out of memory -> drop graphs for good, decode eagerly
        if (f.code != ERR_OOM || !capture_) throw;
        capture_ = false;
        clear();
        return run(src, tgt_lang, max_new, sync_every, eos_mask, use_graph, sl, top);
    }
}

std::vector<std::vector<uint32_t>> GraphCache::run(const Batch &src, uint32_t tgt_lang, int max_new, int sync_every,
                                                   bool eos_mask, bool use_graph, const Shortlist *sl,
                                                   std::vector<std::vector<float>> *top) {
    Model &m = *model_;
    if (!sl) m.ensure_embed();  // the full LM head and input embeddings
    hipStream_t s = m.ctx->stream;
    const ModelConfig &c = m.cfg;
    const bool capture = capture_ && use_graph;
    const int n = src.b, max_m = c.max_position_embeddings;
    const int b = capture ? int(next_pow2(uint32_t(n))) : n;
    const int kb = b, ks = bucket(src.s, 16, max_m), km = bucket(max_new + 2, 32, max_m);
    ++clock_;
    Entry *e = nullptr;
    for (auto &it : entries_)
        if (it.b == kb && it.s == ks && it.m == km && it.sl == sl) e = &it;
    if (!e) {
        Entry ne;
        ne.b = kb;
        ne.s = ks;
        ne.m = km;
        ne.sl = sl;
        ne.st = m.new_state(kb, ks, km, false, false, sl);
        entries_.push_back(std::move(ne));
        e = &entries_.back();
        evict(e);
    }
    e->last_used = clock_;
    StaticState &st = *e->st;
    const int mask_id = eos_mask ? c.eos_token_id : -1;

    std::vector<uint32_t> rows(static_cast<size_t>(n));
    std::iota(rows.begin(), rows.end(), 0u);
    // step 0 consumes decoder_start; its token is replaced by the forced target language.
    // Once the bucket's graph exists these two steps replay it as well (the graph is the
    // same step; the fill and the flag reset between them are ordinary stream work).
    const bool replay = capture && e->exec;
    auto one_step = [&] {
        if (replay) check_hip(hipGraphLaunch(e->exec, s), "graph launch");
        else m.step(st, true, mask_id);
    };
    m.reset_state(st, src, rows, uint32_t(c.decoder_start_token_id));
    one_step();
    check_hip(fill_u32(st.ids, tgt_lang, size_t(st.b), s), "fill");
    if (sl) m.set_shortlist_input(st, tgt_lang);
    std::vector<uint8_t> fin(static_cast<size_t>(st.b));
    for (int r = 0; r < st.b; ++r) fin[r] = r >= n;
    m.ctx->staging.upload(st.finished, fin.data(), fin.size(), s);
    one_step();
    int steps = 2;
    const int max_steps = std::min(max_new + 1, st.m);

    if (capture && !e->exec && steps < max_steps) {
        check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture");
        hipGraph_t graph = nullptr;
        try {
            m.step(st, true, mask_id);
        } catch (...) {
            (void)hipStreamEndCapture(s, &graph);
            if (graph) (void)hipGraphDestroy(graph);
            throw;
        }
        check_hip(hipStreamEndCapture(s, &graph), "end capture");
        hipGraphExec_t exec = nullptr;
        const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        check_hip(ie, "graph instantiate");
        e->exec = exec;
    }
    if (fin_cap_ < size_t(st.b)) {
        if (fin_host_) (void)hipHostFree(fin_host_);
        fin_host_ = nullptr;
        fin_cap_ = 0;
        void *p = nullptr;
        check_hip(hipHostMalloc(&p, size_t(st.b), hipHostMallocDefault), "pinned finished flags");
        fin_host_ = static_cast<uint8_t *>(p);
        fin_cap_ = size_t(st.b);
    }
    if (!fin_ev_) check_hip(hipEventCreateWithFlags(&fin_ev_, hipEventDisableTiming), "event");
    // src/graph.rs:279-288 checks the finished flags every sync_every steps.  Here the
    // flags copied at one check point are read at the next, so the stream keeps
    // sync_every steps queued while the host waits instead of draining.  Steps run
    // after every row has finished only append pad tokens, which the EOS cut below
    // removes, so the output is the same.
    bool pending = false;
    while (steps < max_steps) {
        if (steps % sync_every == 0) {
            if (pending) {
                check_hip(hipEventSynchronize(fin_ev_), "sync");
                if (std::all_of(fin_host_, fin_host_ + st.b, [](uint8_t v) { return v != 0; })) break;
            }
            check_hip(hipMemcpyAsync(fin_host_, st.finished, size_t(st.b), hipMemcpyDeviceToHost, s), "D2H");
            check_hip(hipEventRecord(fin_ev_, s), "event");
            pending = true;
        }
        if (capture && e->exec) check_hip(hipGraphLaunch(e->exec, s), "graph launch");
        else m.step(st, true, mask_id);
        ++steps;
    }
    std::vector<uint32_t> out(static_cast<size_t>(st.b) * st.m);
    std::vector<float> outv(top ? out.size() : 0);
    uint32_t err = 0;
    check_hip(hipMemcpyAsync(out.data(), st.out, out.size() * 4, hipMemcpyDeviceToHost, s), "D2H");
    if (top) check_hip(hipMemcpyAsync(outv.data(), st.outv, outv.size() * 4, hipMemcpyDeviceToHost, s), "D2H");
    check_hip(hipMemcpyAsync(&err, st.err, 4, hipMemcpyDeviceToHost, s), "D2H");
    check_hip(hipStreamSynchronize(s), "sync");
    if (err) fail(ERR_INVALID, kNonFiniteLogits);
    std::vector<std::vector<uint32_t>> res(static_cast<size_t>(n));
    if (top) top->assign(static_cast<size_t>(n), {});
    for (int r = 0; r < n; ++r)
        for (int j = 1; j < steps; ++j) {
            const uint32_t t = out[size_t(r) * st.m + j];
            if (t == uint32_t(c.eos_token_id)) break;
            res[r].push_back(t);
            if (top) (*top)[r].push_back(outv[size_t(r) * st.m + j]);
        }
    return res;
}

// ------------------------------------------------------------------- beam

std::vector<std::vector<uint32_t>> Model::beam(const Batch &src, uint32_t tgt_lang, int max_new, int k, float lp,
                                               bool eos_mask, bool use_graph) {
    // the step writes K/V slot max_new and reads position max_new + pad + 1: both exist
    // only up to max_position_embeddings - 2, the cap translate_batch's budget applies
    if (k < 1 || max_new < 0 || max_new > cfg.max_position_embeddings - 2)
        fail(ERR_INVALID, "beam: max_new " + std::to_string(max_new) + " outside 0.." +
                              std::to_string(cfg.max_position_embeddings - 2) + " or beam size < 1");
    ensure_embed();
    hipStream_t s = ctx->stream;
    const int b = src.b, bk = b * k, V = cfg.vocab_size;
    const uint32_t eos = uint32_t(cfg.eos_token_id);
    const int mask_id = eos_mask ? cfg.eos_token_id : -1;
    // src/translator.rs:195-201: beam search runs Nllb::encode/decode, whose K/V caches
    // (candle KvCache) and cross K/V are f32
    auto st = new_state(bk, src.s, max_new + 2, true, true, nullptr, true);
    std::vector<uint32_t> expand(static_cast<size_t>(bk));
    for (int i = 0; i < bk; ++i) expand[i] = uint32_t(i / k);
    reset_state(*st, src, expand, uint32_t(cfg.decoder_start_token_id));
    // src/model.rs:209-226 reorders every self-attention cache by beam each step.
    // Here the caches stay in place: rows[r][j] names the cache row that holds slot j
    // of beam row r.  Slot j of a cache row is written once (at step j, by that row)
    // and never again, so a reorder only rewrites the map.
    std::vector<uint32_t> rows_map(size_t(bk) * st->m), rows_next(rows_map.size());
    for (int r = 0; r < bk; ++r)
        for (int j = 0; j < st->m; ++j) rows_map[size_t(r) * st->m + j] = uint32_t(r);
    h2d(st->rows, rows_map, s);
    DevTemp tmp;
    float *scratch = tmp.get<float>(logsoftmax_topk_scratch(bk, k) / 4, "topk scratch");
    float *d_vals = tmp.get<float>(size_t(bk) * k, "topk vals");
    uint32_t *d_idx = tmp.get<uint32_t>(size_t(bk) * k, "topk idx");
    // Pinned staging: the per-step copies are asynchronous, and the host waits once per
    // step (for the top-k).  A buffer is rewritten only after that wait, which follows
    // the previous step's copies out of it on the stream.
    struct Pinned {
        void *p = nullptr;
        ~Pinned() {
            if (p) (void)hipHostFree(p);
        }
    } pin_vals, pin_idx, pin_rows, pin_next;
    auto pinned = [&](Pinned &b, size_t bytes) {
        check_hip(hipHostMalloc(&b.p, bytes, hipHostMallocDefault), "pinned staging");
        return b.p;
    };
    float *h_vals = static_cast<float *>(pinned(pin_vals, size_t(bk) * k * 4));
    uint32_t *h_idx = static_cast<uint32_t *>(pinned(pin_idx, size_t(bk) * k * 4));
    uint32_t *h_rows = static_cast<uint32_t *>(pinned(pin_rows, size_t(bk) * st->m * 4));
    uint32_t *h_next = static_cast<uint32_t *>(pinned(pin_next, size_t(bk) * 4));

    auto topk = [&] {
        check_hip(logsoftmax_topk(st->logits, bk, V, k, mask_id, scratch, d_vals, d_idx, s), "topk");
    };
    // Every beam step runs the same launches on the same buffers (ids, rows and the
    // device step counter carry the changes), so one capture of step + top-k is
    // replayed for all steps after the first two.
    const bool capture = use_graph && graphs.capture_enabled();
    struct ExecGuard {
        hipGraphExec_t e = nullptr;
        ~ExecGuard() {
            if (e) (void)hipGraphExecDestroy(e);
        }
    } exec;
    auto advance = [&] {
        if (capture && !exec.e) {
            check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture");
            hipGraph_t graph = nullptr;
            try {
                step(*st, false, mask_id);
                topk();
            } catch (...) {
                (void)hipStreamEndCapture(s, &graph);
                if (graph) (void)hipGraphDestroy(graph);
                throw;
            }
            check_hip(hipStreamEndCapture(s, &graph), "end capture");
            const hipError_t ie = hipGraphInstantiate(&exec.e, graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            check_hip(ie, "graph instantiate");
        }
        if (exec.e) {
            check_hip(hipGraphLaunch(exec.e, s), "graph launch");
        } else {
            step(*st, false, mask_id);
            topk();
        }
    };

    // [start, tgt_lang] fed one position at a time (equal to the t = 2 causal pass)
    step(*st, false, mask_id);
    check_hip(fill_u32(st->ids, tgt_lang, size_t(bk), s), "fill");
    step(*st, false, mask_id);
    topk();

    BeamMerge merge(b, k, max_new, lp, eos);
    const float *vals = h_vals;
    const uint32_t *idx = h_idx;
    for (int stp = 1; stp <= max_new; ++stp) {
        check_hip(hipMemcpyAsync(h_vals, d_vals, size_t(bk) * k * 4, hipMemcpyDeviceToHost, s), "D2H");
        check_hip(hipMemcpyAsync(h_idx, d_idx, size_t(bk) * k * 4, hipMemcpyDeviceToHost, s), "D2H");
        check_hip(hipStreamSynchronize(s), "sync");
        for (int r = 0; r < bk; ++r)  // a row's best log-probability is finite unless its logits are not
            if (!(vals[size_t(r) * k] > -INFINITY)) fail(ERR_INVALID, kNonFiniteLogits);
        if (merge.merge(stp, vals, idx)) break;
        const std::vector<uint32_t> &reorder = merge.reorder(), &next = merge.next();
        // src/model.rs:209-226 gathers the self-attention caches by beam; here only the
        // row map changes (cross K/V and lens are identical within a sentence's beams, and
        // a reorder never leaves a sentence).  Slots 0 .. stp are written; the next step
        // writes slot stp + 1 into row r itself.
        const int m = st->m;
        for (int r = 0; r < bk; ++r) {
            const uint32_t *par = rows_map.data() + size_t(reorder[r]) * m;
            uint32_t *dst = rows_next.data() + size_t(r) * m;
            for (int j = 0; j < m; ++j) dst[j] = j <= stp ? par[j] : uint32_t(r);
        }
        rows_map.swap(rows_next);
        std::copy(rows_map.begin(), rows_map.end(), h_rows);
        std::copy(next.begin(), next.end(), h_next);
        check_hip(hipMemcpyAsync(st->rows, h_rows, rows_map.size() * 4, hipMemcpyHostToDevice, s), "H2D");
        check_hip(hipMemcpyAsync(st->ids, h_next, next.size() * 4, hipMemcpyHostToDevice, s), "H2D");
        advance();
    }
    return merge.result();
}

std::vector<std::vector<uint32_t>> Model::greedy_generic(const Batch &src, uint32_t tgt_lang, int max_new,
                                                         int sync_every, bool eos_mask) {
    if (max_new < 1 || max_new > cfg.max_position_embeddings - 2)
        fail(ERR_INVALID, "greedy: max_new " + std::to_string(max_new) + " outside 1.." +
                              std::to_string(cfg.max_position_embeddings - 2));
    ensure_embed();
    hipStream_t s = ctx->stream;
    const int b = src.b, mask_id = eos_mask ? cfg.eos_token_id : -1;
    auto st = new_state(b, src.s, max_new + 2, false, false, nullptr, true);
    std::vector<uint32_t> rows(static_cast<size_t>(b));
    std::iota(rows.begin(), rows.end(), 0u);
    reset_state(*st, src, rows, uint32_t(cfg.decoder_start_token_id));
    // [start, tgt_lang] fed one position at a time (the t = 2 causal pass of
    // src/translator.rs:228 computes the same); the first position's token is not kept
    step(*st, true, mask_id);
    check_hip(fill_u32(st->ids, tgt_lang, size_t(b), s), "fill");
    std::vector<uint8_t> fin(static_cast<size_t>(b), 0);
    ctx->staging.upload(st->finished, fin.data(), fin.size(), s);
    // step k (1 .. max_new) writes token k into out[:, k]; translator.rs:230-238 stops
    // after max_new tokens or when every row has finished at a multiple of sync_every
    int k = 1;
    for (;; ++k) {
        step(*st, true, mask_id);
        if (k == max_new) break;
        if (k % sync_every == 0) {
            check_hip(hipMemcpyAsync(fin.data(), st->finished, fin.size(), hipMemcpyDeviceToHost, s), "D2H");
            check_hip(hipStreamSynchronize(s), "sync");
            if (std::all_of(fin.begin(), fin.end(), [](uint8_t v) { return v != 0; })) break;
        }
    }
    std::vector<uint32_t> out(size_t(b) * st->m);
    uint32_t err = 0;
    check_hip(hipMemcpyAsync(out.data(), st->out, out.size() * 4, hipMemcpyDeviceToHost, s), "D2H");
    check_hip(hipMemcpyAsync(&err, st->err, 4, hipMemcpyDeviceToHost, s), "D2H");
    check_hip(hipStreamSynchronize(s), "sync");
    if (err) fail(ERR_INVALID, kNonFiniteLogits);
    std::vector<std::vector<uint32_t>> res(static_cast<size_t>(b));
    for (int r = 0; r < b; ++r)
        for (int j = 1; j <= k; ++j) {  // strip (translator.rs:243-246): up to the first EOS
            const uint32_t t = out[size_t(r) * st->m + j];
            if (t == uint32_t(cfg.eos_token_id)) break;
            res[r].push_back(t);
        }
    return res;
}

std::vector<float> Model::teacher_forced(const Batch &src, const std::vector<uint32_t> &tgt, int T, bool kv32) {
    ensure_embed();
    hipStream_t s = ctx->stream;
    const int b = src.b, V = cfg.vocab_size;
    if (T < 1 || int(tgt.size()) != b * T) fail(ERR_INVALID, "teacher_forced: bad target shape");
    if (T + cfg.pad_token_id + 1 >= n_pos) fail(ERR_INVALID, "teacher_forced: sequence longer than the position table");
    for (uint32_t t : tgt)
        if (t >= uint32_t(V)) fail(ERR_INVALID, "token id out of range");
    auto st = new_state(b, src.s, T, true, false, nullptr, kv32);
    std::vector<uint32_t> rows(static_cast<size_t>(b));
    std::iota(rows.begin(), rows.end(), 0u);
    reset_state(*st, src, rows, tgt[0]);
    std::vector<float> out(size_t(b) * T * V);
    std::vector<uint32_t> ids(static_cast<size_t>(b));
    for (int t = 0; t < T; ++t) {
        for (int i = 0; i < b; ++i) ids[i] = tgt[size_t(i) * T + t];
        h2d(st->ids, ids, s);
        step(*st, false, -1);
        for (int i = 0; i < b; ++i)
            check_hip(hipMemcpyAsync(out.data() + (size_t(i) * T + t) * V, st->logits + size_t(i) * V, size_t(V) * 4,
                                     hipMemcpyDeviceToHost, s),
                      "D2H");
        check_hip(hipStreamSynchronize(s), "sync");
    }
    return out;
}

// -------------------------------------------------------------- translator

std::vector<std::vector<uint32_t>> generate_to(Model &m, const std::vector<std::vector<uint32_t>> &src,
                                               uint32_t tgt_lang, const GenOptions &o) {
    if (src.empty()) return {};
    int max_new = 1;
    for (auto &r : src) max_new = std::max(max_new, budget(m.cfg, int(r.size()), o.max_new_tokens));
    // src/translator.rs:184-194: the shortlist serves greedy graph decoding when it holds
    // both forced start tokens
    const Shortlist *sl = o.shortlist.empty() || o.beam_size > 1 || !o.fused ? nullptr : m.shortlist(o.shortlist);
    if (sl && !(sl->contains(uint32_t(m.cfg.decoder_start_token_id)) && sl->contains(tgt_lang))) sl = nullptr;
    auto batch = m.encode(src);
    std::vector<std::vector<uint32_t>> out;
    // src/translator.rs:184-201: greedy with `fused` runs the graph cache (f16 K/V), greedy
    // without it and beam search the generic decoder (f32 K/V)
    if (o.beam_size <= 1 && o.fused)
        out = m.graphs.greedy(*batch, tgt_lang, max_new, std::max(1, o.sync_every), o.eos_mask, true, sl);
    else if (o.beam_size <= 1)
        out = m.greedy_generic(*batch, tgt_lang, max_new, std::max(1, o.sync_every), o.eos_mask);
    else
        out = m.beam(*batch, tgt_lang, max_new, o.beam_size, o.length_penalty, o.eos_mask, o.fused);
    for (size_t i = 0; i < src.size(); ++i) {
        const size_t bud = size_t(budget(m.cfg, int(src[i].size()), o.max_new_tokens));
        if (out[i].size() > bud) out[i].resize(bud);
    }
    return out;
}

std::vector<std::vector<uint32_t>> generate(Model &m, const std::vector<std::vector<uint32_t>> &src, uint32_t tgt_lang,
                                            const GenOptions &o) {
    std::vector<size_t> order(src.size());
    std::iota(order.begin(), order.end(), size_t(0));
    std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return src[a].size() > src[b].size(); });
    std::vector<std::vector<uint32_t>> out(src.size());
    int max_batch = std::max(1, o.max_batch);
    size_t done = 0;
    while (done < order.size()) {
        const size_t end = std::min(order.size(), done + size_t(max_batch));
        std::vector<std::vector<uint32_t>> batch;
        for (size_t i = done; i < end; ++i) batch.push_back(src[order[i]]);
        std::vector<std::vector<uint32_t>> ids;
        try {
            ids = generate_to(m, batch, tgt_lang, o);
        } catch (const Failure &f) {
            // src/translator.rs:150-158: free cached buffers, retry with smaller batches
            // ... unless the full-vocabulary LM head itself does not fit (translator.rs:152)
            if (f.code == ERR_OOM && max_batch > 1 && f.msg.find("full-vocabulary") == std::string::npos) {
                max_batch /= 2;
                m.graphs.clear();
                continue;
            }
            throw;
        }
        for (size_t i = done; i < end; ++i) out[order[i]] = std::move(ids[i - done]);
        done = end;
    }
    return out;
}

}  // namespace mlg
