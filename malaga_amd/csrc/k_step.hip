// Fused decoder-step kernels for batch <= 4 (src/model.rs:552-612 with the
// fused kernels of kernels/malaga.cu folded into the projections).
//
// One layer is six launches instead of twelve:
//   qkv       : [embedding +] residual + LayerNorm -> GEMV -> q | f16 K/V at slot *step
//   attn_out  : self-attention over the f16 cache   -> GEMV (+bias)
//   cross_q   : residual + LayerNorm                -> GEMV (+bias)
//   cross_out : cross-attention over the encoder K/V -> GEMV (+bias)
//   up        : residual + LayerNorm                -> GEMV (+bias, ReLU)
//   down      : GEMV over the FFN activations (+bias)
// Every workgroup computes its prologue (the LayerNorm or the attention of all
// heads) redundantly in LDS: at decode sizes that costs a few KB of L2 reads and
// saves a launch plus a round trip through HBM per fused op.  The first row
// group's weights are requested before the prologue starts.  Workgroup 0 writes
// the updated residual stream to the other half of a ping-pong pair.
#include "dequant.hpp"
#include "gemv_core.hpp"
#include "kernels.hpp"

namespace mlg {

namespace {

enum Pro : int { PRO_EMBED = 0, PRO_RESID = 1, PRO_ATTN = 2, PRO_GLOBAL = 3 };
enum Epi : int { EPI_STORE = 0, EPI_QKV = 1 };

struct StepArgs {
    WPtr w;
    GemvGeom g;
    int nb;  // rows of the state
    int d;   // model width (prologue vector length for EMBED / RESID / ATTN)
    // prologue inputs
    const float *x_in, *y_in;  // RESID: x = x_in + y_in
    float *x_out;              // RESID / EMBED: new residual stream (written by workgroup 0)
    const float *gamma, *beta;
    float eps;
    const uint8_t *eq, *es, *ed;  // EMBED: token embedding planes
    const uint32_t *ids;
    const float *pos;
    uint32_t pos_base;
    float emb_scale;
    const float *q;                 // ATTN: queries [nb][d]
    const __half *K, *V;            // ATTN: [nb][H][L][hd]
    int H, hd, L;
    const uint32_t *lens;           // ATTN: cross lengths, or null -> *step + 1
    const uint32_t *step;
    const float *xg;                // GLOBAL: x [nb][ldx]
    int ldx;
    // epilogue
    const float *bias;
    int relu;
    float *y;  // EPI_STORE: [nb][N]
    float *qo;                  // EPI_QKV: q [nb][d]
    __half *kc, *vc;            // EPI_QKV: caches [nb][H][m][hd]
    int m;
};

__device__ __forceinline__ void block_sums(float (&v)[4], int n, float *red) {
    // sums n (<= 4) values over the 256-thread workgroup; red holds >= 16 floats
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (i < n) v[i] = wave_sum(v[i]);
    if (lane == 0)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < n) red[i * 4 + w] = v[i];
    lds_barrier();
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (i < n) v[i] = red[i * 4] + red[i * 4 + 1] + red[i * 4 + 2] + red[i * 4 + 3];
    lds_barrier();
}

// LayerNorm of the nb rows of xs[nb][d] (LDS) in place, biased variance.  gamma and
// beta (d <= 4096: 16 values per thread) are fetched before the reductions.
__device__ __forceinline__ void ln_lds(float *xs, int nb, int d, const float *gamma, const float *beta, float eps,
                                       float *red) {
    float gr[16], br[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int k = threadIdx.x + i * 256;
        gr[i] = k < d ? gamma[k] : 0.f;
        br[i] = k < d ? beta[k] : 0.f;
    }
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    for (int bi = 0; bi < nb; ++bi)
        for (int k = threadIdx.x; k < d; k += 256) s[bi] += xs[bi * d + k];
    block_sums(s, nb, red);
    float mean[4], v2[4] = {0.f, 0.f, 0.f, 0.f};
    for (int bi = 0; bi < nb; ++bi) {
        mean[bi] = s[bi] / float(d);
        for (int k = threadIdx.x; k < d; k += 256) {
            const float c = xs[bi * d + k] - mean[bi];
            v2[bi] += c * c;
        }
    }
    block_sums(v2, nb, red);
    for (int bi = 0; bi < nb; ++bi) {
        const float rstd = rsqrtf(v2[bi] / float(d) + eps);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int k = threadIdx.x + i * 256;
            if (k < d) xs[bi * d + k] = (xs[bi * d + k] - mean[bi]) * rstd * gr[i] + br[i];
        }
    }
    lds_barrier();
}

template <int ET>
__device__ __forceinline__ void embed_rows(const StepArgs &a, float *xs) {
    const uint32_t s = *a.step;
    for (int bi = 0; bi < a.nb; ++bi) {
        const uint32_t tok = a.ids[bi];
        const float *pr = a.pos + size_t(s + a.pos_base) * a.d;
        for (int k0 = threadIdx.x * 16; k0 < a.d; k0 += 256 * 16) {
            float e[16];
            dequant16<ET>(a.eq, a.es, a.ed, a.d, int(tok), k0, e);
#pragma unroll
            for (int i = 0; i < 16; ++i) xs[bi * a.d + k0 + i] = e[i] * a.emb_scale + pr[k0 + i];
        }
    }
}

// Attention of all (row, head) pairs into out[nb][H*HD] (LDS).  Scores live in
// sc[nb*H][L], queries are staged in qs[nb][d], key-split partial sums in
// part[2048] (all LDS).  nb * H must divide 256 and be >= 4.  Every phase spreads
// (pair, key) work over the whole workgroup and issues several independent
// 16-byte loads per thread before using them.
template <int HD>
__device__ __forceinline__ void attention_lds(const StepArgs &a, float *qs, float *sc, float *part, float *out,
                                              float *red) {
    const int H = a.H, d = a.d, L = a.L, nb = a.nb;
    const int pairs = nb * H;
    int nmax = 0;
    const int n_self = a.lens ? 0 : int(*a.step) + 1;
    for (int bi = 0; bi < nb; ++bi) nmax = max(nmax, a.lens ? int(a.lens[bi]) : n_self);
    // phase 1: scores, item f -> (pair f / nmax, key f % nmax), 4 items per thread in
    // flight; the first keys are requested before the queries are staged in LDS
    constexpr int U = 4;
    const int items = pairs * nmax;
    bool staged = false;
    for (int base = threadIdx.x; base < items || !staged; base += 256 * U) {
        uint4 kr[U][HD / 8];
        int fp[U], fj[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int f = base + u * 256;
            fp[u] = f / nmax;
            fj[u] = f % nmax;
            const int bi = min(fp[u], pairs - 1) / H;
            const int n = a.lens ? int(a.lens[bi]) : n_self;
            ok[u] = f < items && fj[u] < n;
            const int p = ok[u] ? fp[u] : 0, j = ok[u] ? fj[u] : 0;
            const uint4 *k8 = reinterpret_cast<const uint4 *>(a.K + (size_t(p) * L + j) * HD);
#pragma unroll
            for (int t = 0; t < HD / 8; ++t) kr[u][t] = k8[t];
        }
        if (!staged) {  // uniform: the first trip of every thread
            for (int i = threadIdx.x * 4; i < nb * d; i += 256 * 4)
                *reinterpret_cast<float4 *>(qs + i) = *reinterpret_cast<const float4 *>(a.q + i);
            lds_barrier();
            staged = true;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (!ok[u]) continue;
            const int bi = fp[u] / H, hh = fp[u] % H;
            const float *qv = qs + bi * d + hh * HD;
            float acc = 0.f;
#pragma unroll
            for (int t = 0; t < HD / 8; ++t) {
                const uint32_t wv[4] = {kr[u][t].x, kr[u][t].y, kr[u][t].z, kr[u][t].w};
#pragma unroll
                for (int q2 = 0; q2 < 4; ++q2) {
                    acc = fmaf(h2f(wv[q2]), qv[8 * t + 2 * q2], acc);
                    acc = fmaf(h2f(wv[q2] >> 16), qv[8 * t + 2 * q2 + 1], acc);
                }
            }
            sc[fp[u] * L + fj[u]] = acc;
        }
    }
    lds_barrier();
    // phase 2: softmax per pair, 256 / pairs threads per pair (a power of two <= 64)
    const int tpp = 256 / pairs;
    {
        const int p = threadIdx.x / tpp, sub = threadIdx.x % tpp;
        const int n = a.lens ? int(a.lens[p / H]) : n_self;
        float mx = -INFINITY, sum = 0.f;
        for (int j = sub; j < n; j += tpp) mx = fmaxf(mx, sc[p * L + j]);
        for (int o = tpp >> 1; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        for (int j = sub; j < n; j += tpp) {
            const float e = expf(sc[p * L + j] - mx);
            sc[p * L + j] = e;
            sum += e;
        }
        for (int o = tpp >> 1; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
        if (sub == 0) red[16 + p] = 1.f / sum;
    }
    lds_barrier();
    // phase 3: P.V, work item -> (pair, 8 consecutive dims, key split); 8 keys in flight
    constexpr int G = HD / 8;
    const int groups8 = pairs * G;
    const int splits = max(1, 256 / groups8);
    for (int it = threadIdx.x; it < groups8 * splits; it += 256) {
        const int gi = it % groups8, sp = it / groups8;
        const int p = gi / G, e0 = (gi % G) * 8;
        const int bi = p / H;
        const int n = a.lens ? int(a.lens[bi]) : n_self;
        const __half *Vb = a.V + size_t(p) * L * HD + e0;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int j0 = sp; j0 < n; j0 += 8 * splits) {
            uint4 raw[8];
            float pj[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int j = j0 + u * splits;
                const int jj = j < n ? j : sp;
                raw[u] = *reinterpret_cast<const uint4 *>(Vb + size_t(jj) * HD);
                pj[u] = j < n ? sc[p * L + jj] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t wv[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
                for (int q2 = 0; q2 < 4; ++q2) {
                    acc[2 * q2] = fmaf(pj[u], h2f(wv[q2]), acc[2 * q2]);
                    acc[2 * q2 + 1] = fmaf(pj[u], h2f(wv[q2] >> 16), acc[2 * q2 + 1]);
                }
            }
        }
        if (splits == 1) {
            const float inv = red[16 + p];
            const int hh = p % H;
#pragma unroll
            for (int u = 0; u < 8; ++u) out[bi * d + hh * HD + e0 + u] = acc[u] * inv;
        } else {
#pragma unroll
            for (int u = 0; u < 8; ++u) part[(sp * groups8 + gi) * 8 + u] = acc[u];
        }
    }
    lds_barrier();
    if (splits > 1) {
        for (int i = threadIdx.x; i < groups8 * 8; i += 256) {
            const int g = i / 8, u = i % 8;
            float o = 0.f;
            for (int s2 = 0; s2 < splits; ++s2) o += part[(s2 * groups8 + g) * 8 + u];
            const int pp = g / G, ee = (g % G) * 8 + u;
            const int bi = pp / H, hh = pp % H;
            out[bi * d + hh * HD + ee] = o * red[16 + pp];
        }
        lds_barrier();
    }
}

template <int T, int B, int CPL, int PRO, int EPI, int ET>
__global__ __launch_bounds__(256) void k_step(StepArgs a) {
    constexpr int XW = GTraits<T>::XW, NS = GTraits<T>::NS;
    extern __shared__ float lds[];
    __shared__ float red[96];
    const int lane = threadIdx.x & 63;
    const int cl = lane & ((1 << a.g.lpr_log2) - 1);
    const int gwave = blockIdx.x * 4 + (threadIdx.x >> 6), nwaves = gridDim.x * 4;
    float xr[CPL][B][XW], xs[CPL][B][NS];

    auto prologue = [&] {
        if constexpr (PRO == PRO_GLOBAL) {
            gemv_load_x<T, B, CPL>(a.xg, a.ldx, a.nb, a.g, cl, xr, xs);
        } else if constexpr (PRO == PRO_ATTN) {
            float *qs = lds, *out = lds + a.nb * a.d, *part = lds + 2 * a.nb * a.d, *sc = part + 2048;
            if (a.hd == 64) attention_lds<64>(a, qs, sc, part, out, red);
            else if (a.hd == 128) attention_lds<128>(a, qs, sc, part, out, red);
            else attention_lds<16>(a, qs, sc, part, out, red);
            gemv_load_x<T, B, CPL>(out, a.d, a.nb, a.g, cl, xr, xs);
        } else {
            float *v = lds;
            if constexpr (PRO == PRO_EMBED) {
                embed_rows<ET>(a, v);
            } else {
                for (int i = threadIdx.x * 4; i < a.nb * a.d; i += 256 * 4) {
                    const float4 xa = *reinterpret_cast<const float4 *>(a.x_in + i);
                    const float4 ya = *reinterpret_cast<const float4 *>(a.y_in + i);
                    *reinterpret_cast<float4 *>(v + i) = make_float4(xa.x + ya.x, xa.y + ya.y, xa.z + ya.z, xa.w + ya.w);
                }
            }
            lds_barrier();
            if (blockIdx.x == 0)
                for (int i = threadIdx.x; i < a.nb * a.d; i += 256) a.x_out[i] = v[i];
            lds_barrier();
            ln_lds(v, a.nb, a.d, a.gamma, a.beta, a.eps, red);
            gemv_load_x<T, B, CPL>(v, a.d, a.nb, a.g, cl, xr, xs);
        }
    };

    if constexpr (EPI == EPI_STORE) {
        auto epi = [&](int row, int bi, float v) {
            if (bi >= a.nb) return;
            if (a.relu) v = fmaxf(v, 0.f);
            a.y[size_t(bi) * a.w.N + row] = v;
        };
        gemv_rows<T, B, CPL>(a.w, a.g, xr, xs, gwave, nwaves, prologue, epi, a.bias);
    } else {
        const uint32_t slot = *a.step;
        auto epi = [&](int row, int bi, float v) {
            if (bi >= a.nb) return;
            const int d = a.d;
            if (row < d) {
                a.qo[size_t(bi) * d + row] = v;
            } else {
                const int c = row < 2 * d ? row - d : row - 2 * d;
                const size_t off = ((size_t(bi) * a.H + c / a.hd) * a.m + slot) * a.hd + c % a.hd;
                (row < 2 * d ? a.kc : a.vc)[off] = __float2half(v);
            }
        };
        gemv_rows<T, B, CPL>(a.w, a.g, xr, xs, gwave, nwaves, prologue, epi, a.bias);
    }
}

template <int T, int B, int CPL, int PRO, int EPI, int ET>
hipError_t launch_t(const StepArgs &a, int grid, size_t lds, hipStream_t st) {
    if constexpr (GTraits<T>::XW * B * CPL > kGemvMaxXRegs) {
        return hipErrorInvalidValue;
    } else {
        hipLaunchKernelGGL((k_step<T, B, CPL, PRO, EPI, ET>), dim3(grid), dim3(256), lds, st, a);
        return hipGetLastError();
    }
}

template <int T, int PRO, int EPI, int ET>
hipError_t dispatch_bc(const StepArgs &a, int B, int cpl, int grid, size_t lds, hipStream_t st) {
#define MLG_CASE(BB, CC) \
    if (B == BB && cpl == CC) return launch_t<T, BB, CC, PRO, EPI, ET>(a, grid, lds, st);
    MLG_CASE(1, 1) MLG_CASE(1, 2) MLG_CASE(2, 1) MLG_CASE(2, 2) MLG_CASE(4, 1)
#undef MLG_CASE
    return hipErrorInvalidValue;
}

template <int PRO, int EPI, int ET>
hipError_t dispatch_t(uint32_t type, const StepArgs &a, int B, int cpl, int grid, size_t lds, hipStream_t st) {
    switch (type) {
    case GGML_Q4_K: return dispatch_bc<GGML_Q4_K, PRO, EPI, ET>(a, B, cpl, grid, lds, st);
    case GGML_Q5_K: return dispatch_bc<GGML_Q5_K, PRO, EPI, ET>(a, B, cpl, grid, lds, st);
    case GGML_Q6_K: return dispatch_bc<GGML_Q6_K, PRO, EPI, ET>(a, B, cpl, grid, lds, st);
    case GGML_Q8_0: return dispatch_bc<GGML_Q8_0, PRO, EPI, ET>(a, B, cpl, grid, lds, st);
    case GGML_F16: return dispatch_bc<GGML_F16, PRO, EPI, ET>(a, B, cpl, grid, lds, st);
    case GGML_F32: return dispatch_bc<GGML_F32, PRO, EPI, ET>(a, B, cpl, grid, lds, st);
    default: return hipErrorInvalidValue;
    }
}

bool prepare(const DevMatrix &w, int nb, StepArgs &a, int *cpl) {
    if (nb < 1 || nb > 4 || nb > gemv_max_batch(w) || !gemv_geometry(w, &a.g, cpl)) return false;
    a.w = wptr_of(w);
    a.nb = nb;
    return true;
}

}  // namespace

size_t step_attn_lds(int nb, int d, int H, int L) {
    return sizeof(float) * (size_t(2) * nb * d + 2048 + size_t(nb) * H * L);
}

bool step_fusable(const DevMatrix &w, int nb, int d, int H, int hd, int L) {
    GemvGeom g;
    int cpl;
    if (nb < 1 || nb > 4 || nb > gemv_max_batch(w) || !gemv_geometry(w, &g, &cpl) || cpl > 2) return false;
    if (nb == 4 && cpl > 1) return false;
    if ((hd != 16 && hd != 64 && hd != 128) || d % 16 || nb * H < 4 || nb * H > 64 || 256 % (nb * H)) return false;
    // attention scores + staged queries + outputs must fit the LDS budget
    // dynamic LDS (+ 384 B static) within the default 64 KB per workgroup
    return step_attn_lds(nb, d, H, L) + 512 <= 64 * 1024 && size_t(nb) * d * 4 + 512 <= 64 * 1024;
}

hipError_t step_qkv(const DevMatrix &w, const float *bias, int nb, int d, const DevMatrix *emb, const uint32_t *ids, const float *pos, uint32_t pos_base, float emb_scale,
                    const float *x_in, const float *y_in, float *x_out, const float *gamma, const float *beta,
                    float eps, const uint32_t *step, float *q, __half *kc, __half *vc, int H, int hd, int m,
                    hipStream_t st) {
    StepArgs a{};
    int cpl;
    if (!prepare(w, nb, a, &cpl)) return hipErrorInvalidValue;
    a.d = d;
    a.x_in = x_in;
    a.y_in = y_in;
    a.x_out = x_out;
    a.gamma = gamma;
    a.beta = beta;
    a.eps = eps;
    if (emb) {
        a.eq = emb->q;
        a.es = emb->s;
        a.ed = emb->d;
    }
    a.ids = ids;
    a.pos = pos;
    a.pos_base = pos_base;
    a.emb_scale = emb_scale;
    a.step = step;
    a.bias = bias;
    a.qo = q;
    a.kc = kc;
    a.vc = vc;
    a.H = H;
    a.hd = hd;
    a.m = m;
    const size_t lds = sizeof(float) * size_t(nb) * d;
    const int grid = gemv_grid(w);
    const int B = gemv_round_b(nb);
    if (!emb) return dispatch_t<PRO_RESID, EPI_QKV, GGML_F32>(w.type, a, B, cpl, grid, lds, st);
    // (projection type, embedding type) pairs the presets produce (src/convert.rs:188-211)
    const uint32_t t = w.type, e = emb->type;
    if (t == GGML_Q4_K && e == GGML_Q6_K) return dispatch_bc<GGML_Q4_K, PRO_EMBED, EPI_QKV, GGML_Q6_K>(a, B, cpl, grid, lds, st);
    if (t == GGML_Q5_K && e == GGML_Q6_K) return dispatch_bc<GGML_Q5_K, PRO_EMBED, EPI_QKV, GGML_Q6_K>(a, B, cpl, grid, lds, st);
    if (t == GGML_Q6_K && e == GGML_Q6_K) return dispatch_bc<GGML_Q6_K, PRO_EMBED, EPI_QKV, GGML_Q6_K>(a, B, cpl, grid, lds, st);
    if (t == GGML_Q8_0 && e == GGML_Q8_0) return dispatch_bc<GGML_Q8_0, PRO_EMBED, EPI_QKV, GGML_Q8_0>(a, B, cpl, grid, lds, st);
    if (t == GGML_F16 && e == GGML_F16) return dispatch_bc<GGML_F16, PRO_EMBED, EPI_QKV, GGML_F16>(a, B, cpl, grid, lds, st);
    if (t == GGML_F32 && e == GGML_F32) return dispatch_bc<GGML_F32, PRO_EMBED, EPI_QKV, GGML_F32>(a, B, cpl, grid, lds, st);
    return hipErrorInvalidValue;
}

bool step_embed_supported(uint32_t t, uint32_t e) {
    return (e == GGML_Q6_K && (t == GGML_Q4_K || t == GGML_Q5_K || t == GGML_Q6_K)) ||
           (t == e && (t == GGML_Q8_0 || t == GGML_F16 || t == GGML_F32));
}

hipError_t step_attn_proj(const DevMatrix &w, const float *bias, int nb, int d, const float *q, const __half *K,
                          const __half *V, int H, int hd, int L, const uint32_t *lens, const uint32_t *step, float *y,
                          hipStream_t st) {
    StepArgs a{};
    int cpl;
    if (!prepare(w, nb, a, &cpl)) return hipErrorInvalidValue;
    a.d = d;
    a.q = q;
    a.K = K;
    a.V = V;
    a.H = H;
    a.hd = hd;
    a.L = L;
    a.lens = lens;
    a.step = step;
    a.bias = bias;
    a.y = y;
    return dispatch_t<PRO_ATTN, EPI_STORE, GGML_F32>(w.type, a, gemv_round_b(nb), cpl, gemv_grid(w),
                                                       step_attn_lds(nb, d, H, L), st);
}

hipError_t step_resid_proj(const DevMatrix &w, const float *bias, bool relu, int nb, int d, const float *x_in,
                           const float *y_in, float *x_out, const float *gamma, const float *beta, float eps, float *y,
                           hipStream_t st) {
    StepArgs a{};
    int cpl;
    if (!prepare(w, nb, a, &cpl)) return hipErrorInvalidValue;
    a.d = d;
    a.x_in = x_in;
    a.y_in = y_in;
    a.x_out = x_out;
    a.gamma = gamma;
    a.beta = beta;
    a.eps = eps;
    a.bias = bias;
    a.relu = relu ? 1 : 0;
    a.y = y;
    return dispatch_t<PRO_RESID, EPI_STORE, GGML_F32>(w.type, a, gemv_round_b(nb), cpl, gemv_grid(w),
                                                        sizeof(float) * size_t(nb) * d, st);
}

hipError_t step_proj(const DevMatrix &w, const float *bias, int nb, const float *x, float *y, hipStream_t st) {
    StepArgs a{};
    int cpl;
    if (!prepare(w, nb, a, &cpl)) return hipErrorInvalidValue;
    a.xg = x;
    a.ldx = w.K;
    a.bias = bias;
    a.y = y;
    return dispatch_t<PRO_GLOBAL, EPI_STORE, GGML_F32>(w.type, a, gemv_round_b(nb), cpl, gemv_grid(w), 0, st);
}

}  // namespace mlg
