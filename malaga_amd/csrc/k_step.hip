// Fused decoder-step kernels for batch <= 4 (src/model.rs:552-612, with the
// fused kernels of kernels/malaga.cu folded into the projections).
//
// One layer is six launches:
//   qkv        : [embedding |] residual + LayerNorm -> GEMV -> q | f16 K/V at slot *step
//   attn_head  : per group of heads: attention over the f16 cache, then the group's
//                column slice of the out-projection -> one partial sum per group
//   resid_proj : residual (x + partial sums + bias) + LayerNorm -> GEMV
//                (cross_q; then, after the cross attn_head, ffn_up with ReLU)
//   proj       : GEMV over the FFN activations (ffn_down)
// The residual prologue keeps each thread's values in registers: residual,
// partial sums, gamma and beta are requested together, after the first row
// group's weights.  Workgroup 0 writes the updated residual stream to the other
// half of a ping-pong pair.  Partial sums are added in a fixed order, so results
// do not depend on scheduling.
#include "dequant.hpp"
#include "gemv_core.hpp"
#include "kernels.hpp"

namespace mlg {

namespace {

enum Pro : int { PRO_EMBED = 0, PRO_RESID = 1, PRO_GLOBAL = 2, PRO_RESID_PRE = 3 };
enum Epi : int { EPI_STORE = 0, EPI_QKV = 1 };

constexpr int kMaxF4 = 4;  // float4 slots per thread and row in the residual prologue (d <= 4096)

struct StepArgs {
    WPtr w;
    GemvGeom g;
    int nb;  // rows of the state
    int d;   // model width
    // residual prologue: x = x_in + sum_{p < P} part[p] + pbias
    const float *x_in;
    const float *part;  // [P][nb][d]
    int P;
    const float *pbias;  // bias of the projection that produced the partials (or null)
    float *x_out;        // new residual stream (workgroup 0 writes it)
    const float *gamma, *beta;
    float eps;
    // embedding prologue: x = E[ids[r]] * emb_scale + pos[*step + pos_base]
    const uint8_t *eq, *es, *ed;
    const uint32_t *ids;
    uint32_t elast;  // last row of the embedding: device-produced ids are clamped to it
    // ... or, where src_row[r] != kNoRow, x = src_emb[r][src_row[r]] * emb_scale + pos (a copied source token)
    const float *src_emb;
    const uint32_t *src_row;
    int S;
    const float *pos;
    uint32_t pos_base;
    float emb_scale;
    const uint32_t *step;
    // plain prologue: x [nb][ldx] in global memory
    const float *xg;
    int ldx;
    // epilogue
    const float *bias;
    int relu;
    float *y;         // EPI_STORE: [nb][N]
    float *qo;        // EPI_QKV: q [nb][d]
    __half *kc, *vc;  // EPI_QKV: caches [nb][H][m][hd]
    int H, hd, m;
};

constexpr int kPreParts = 8;  // partial sums a preloading residual prologue keeps in registers

// Operands of the residual prologue, loaded before the weights when they fit
// (rows <= 2, one float4 slot per row, P <= kPreParts).
template <int R = 2>
struct PreLoadsR {
    float4 part[R][kPreParts], x[R], pb, gr, br;
};
using PreLoads = PreLoadsR<2>;

template <int R = 2>
__device__ __forceinline__ void preload(const StepArgs &a, PreLoadsR<R> &L) {
    // every load unconditional (partials past a.P and rows past nb read a valid one,
    // never used): a skipped load would leave the compiler unsure of the order of the
    // loads issued after these, and the prologue would wait for them too
    const int f = min(int(threadIdx.x), (a.d >> 2) - 1);
#pragma unroll
    for (int bi = 0; bi < R; ++bi) {
        const int bc = min(bi, a.nb - 1);
#pragma unroll
        for (int p = 0; p < kPreParts; ++p) L.part[bi][p] = ld4(a.part + (size_t(min(p, a.P - 1)) * a.nb + bc) * a.d, f);
        L.x[bi] = ld4(a.x_in + size_t(bc) * a.d, f);
    }
    L.pb = ld4(a.pbias ? a.pbias : a.gamma, f);  // used only with a.pbias
    L.gr = ld4(a.gamma, f);
    L.br = ld4(a.beta, f);
}

// LayerNorm of the rows held in registers (thread t owns float4 slots t, t + 256,
// ... of each row), written to xs[nb][d] (LDS).  Mean and variance come from one
// pass of f64 sums of x and x^2 (biased variance).
// NW: waves of the workgroup (red holds 2 * 4 * NW doubles); waves past the first
// four hold no slots and add zeros.
// MF: float4 slots per thread and row (d <= 1024 MF).
template <int NW = 4, int MF = kMaxF4>
__device__ __forceinline__ void ln_to_lds(const float4 (&v)[4][MF], const float4 (&gr)[MF], const float4 (&br)[MF],
                                          int nb, int d, float eps, float *xs, double *red) {
    const int t = threadIdx.x, nf = d >> 2, lane = t & 63, w = t >> 6;
    double s1[4] = {0.0, 0.0, 0.0, 0.0}, s2[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int c = 0; c < MF; ++c)
            if (bi < nb && t + 256 * c < nf) {
                const double x0 = v[bi][c].x, x1 = v[bi][c].y, x2 = v[bi][c].z, x3 = v[bi][c].w;
                s1[bi] += (x0 + x1) + (x2 + x3);
                s2[bi] += (x0 * x0 + x1 * x1) + (x2 * x2 + x3 * x3);
            }
#pragma unroll
    for (int bi = 0; bi < 4; ++bi)
        if (bi < nb) {
            s1[bi] = wave_sum_f64(s1[bi]);
            s2[bi] = wave_sum_f64(s2[bi]);
            if (lane == 0) {
                red[(2 * bi) * NW + w] = s1[bi];
                red[(2 * bi + 1) * NW + w] = s2[bi];
            }
        }
    lds_barrier();
    // fixed-order sums; the zeros of waves 4.. leave the 4-wave value unchanged
    auto sum_nw = [](const double *r) {
        double q = (r[0] + r[1]) + (r[2] + r[3]);
#pragma unroll
        for (int k = 4; k < NW; k += 4) q += (r[k] + r[k + 1]) + (r[k + 2] + r[k + 3]);
        return q;
    };
#pragma unroll
    for (int bi = 0; bi < 4; ++bi) {
        if (bi >= nb) break;
        const double *r1 = red + 2 * bi * NW, *r2 = r1 + NW;
        const double mean = sum_nw(r1) / d;
        const double var = fmax(sum_nw(r2) / d - mean * mean, 0.0);
        const float rstd = float(1.0 / sqrt(var + double(eps))), m = float(mean);
#pragma unroll
        for (int c = 0; c < MF; ++c)
            if (t + 256 * c < nf)
                *reinterpret_cast<float4 *>(xs + bi * lds_pad(d) + lds_pad(4 * (t + 256 * c))) =
                    make_float4((v[bi][c].x - m) * rstd * gr[c].x + br[c].x, (v[bi][c].y - m) * rstd * gr[c].y + br[c].y,
                                (v[bi][c].z - m) * rstd * gr[c].z + br[c].z, (v[bi][c].w - m) * rstd * gr[c].w + br[c].w);
    }
    lds_barrier();
}

// Builds the residual stream x (PRO_RESID / PRO_RESID_PRE) or the embedded tokens
// (PRO_EMBED) in registers, writes it to x_out (workgroup 0) and leaves
// LayerNorm(x) in xs[nb][d] (LDS).
template <int PRO, int ET, int NW = 4, int MF = kMaxF4, int PR = 2>
__device__ __forceinline__ void resid_ln_prologue(const StepArgs &a, const PreLoadsR<PR> &L, float *xs,
                                                  double *red) {
    const int d = a.d, nb = a.nb, nf = d >> 2, nc = (nf + 255) >> 8;
    const int t = threadIdx.x;
    float4 v[4][MF], gr[MF], br[MF];
    if constexpr (PRO == PRO_RESID_PRE) {
        gr[0] = L.gr;
        br[0] = L.br;
#pragma unroll
        for (int bi = 0; bi < PR; ++bi) {
            if (bi >= nb) break;
            float4 acc = L.part[bi][0];
#pragma unroll
            for (int p = 1; p < kPreParts; ++p)
                if (p < a.P) add4(acc, L.part[bi][p]);
            if (a.pbias) add4(acc, L.pb);
            v[bi][0] = make_float4(L.x[bi].x + acc.x, L.x[bi].y + acc.y, L.x[bi].z + acc.z, L.x[bi].w + acc.w);
        }
    } else {
#pragma unroll
        for (int c = 0; c < MF; ++c) {
            if (c >= nc) break;
            const int f = min(t + 256 * c, nf - 1);
            gr[c] = ld4(a.gamma, f);
            br[c] = ld4(a.beta, f);
        }
        if constexpr (PRO == PRO_EMBED) {
            const uint32_t s = *a.step;
            const float *pr = a.pos + size_t(s + a.pos_base) * d;
            const int per_row = d >> 4;
            for (int i = t; i < nb * per_row; i += 256) {
                const int bi = i / per_row, k0 = (i % per_row) * 16;
                float e[16];
                const uint32_t sr = a.src_row ? a.src_row[bi] : kNoRow;
                if (sr != kNoRow) {
                    const float *er = a.src_emb + (size_t(bi) * a.S + sr) * d + k0;
#pragma unroll
                    for (int j = 0; j < 16; ++j) e[j] = er[j];
                } else {
                    dequant16<ET>(a.eq, a.es, a.ed, d, int(min(a.ids[bi], a.elast)), k0, e);
                }
#pragma unroll
                for (int j = 0; j < 16; ++j) xs[bi * lds_pad(d) + lds_pad(k0 + j)] = e[j] * a.emb_scale + pr[k0 + j];
            }
            lds_barrier();
#pragma unroll
            for (int bi = 0; bi < 4; ++bi) {
                if (bi >= nb) break;
#pragma unroll
                for (int c = 0; c < MF; ++c)
                    if (c < nc)
                        v[bi][c] = *reinterpret_cast<const float4 *>(xs + bi * lds_pad(d) +
                                                                     lds_pad(4 * min(t + 256 * c, nf - 1)));
            }
        } else {
#pragma unroll
            for (int bi = 0; bi < 4; ++bi) {
                if (bi >= nb) break;
#pragma unroll
                for (int c = 0; c < MF; ++c) {
                    if (c >= nc) break;
                    const int f = min(t + 256 * c, nf - 1);
                    float4 acc = ld4(a.part + size_t(bi) * d, f);
                    for (int p = 1; p < a.P; ++p) add4(acc, ld4(a.part + (size_t(p) * nb + bi) * d, f));
                    if (a.pbias) add4(acc, ld4(a.pbias, f));
                    const float4 x = ld4(a.x_in + size_t(bi) * d, f);
                    v[bi][c] = make_float4(x.x + acc.x, x.y + acc.y, x.z + acc.z, x.w + acc.w);
                }
            }
        }
    }
    if (blockIdx.x == 0 && blockIdx.y == 0) {
#pragma unroll
        for (int bi = 0; bi < 4; ++bi)
#pragma unroll
            for (int c = 0; c < MF; ++c)
                if (bi < nb && t + 256 * c < nf)
                    reinterpret_cast<float4 *>(a.x_out + size_t(bi) * d)[t + 256 * c] = v[bi][c];
    }
    ln_to_lds<NW, MF>(v, gr, br, nb, d, a.eps, xs, red);
}

template <int T, int B, int CPL, int PRO, int EPI, int ET>
__global__ __launch_bounds__(256) void k_step(StepArgs a) {
    extern __shared__ float lds[];
    __shared__ double red[32];
    const int lane = threadIdx.x & 63;
    const int cl = lane & ((1 << a.g.lpr_log2) - 1);
    // a scalar: the per-step branches on it stay uniform (no divergent load paths)
    const int gwave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6)), nwaves = gridDim.x * 4;
    // f32 x: these kernels are latency-bound, and staging integer limbs of x would
    // add a conversion and a barrier to the critical path (measured slower)
    XF<T, B> xr[CPL];
    PreLoads L;

    auto pre = [&] {
        if constexpr (PRO == PRO_RESID_PRE) preload(a, L);
    };
    auto prologue = [&] {
        if constexpr (PRO == PRO_GLOBAL) {
            gemv_load_x<T, B, CPL>(a.xg, a.ldx, a.nb, a.g, cl, xr);
        } else {
            resid_ln_prologue<PRO, ET>(a, L, lds, red);
            gemv_load_x<T, B, CPL, true>(lds, lds_pad(a.d), a.nb, a.g, cl, xr);
        }
    };

    if constexpr (EPI == EPI_STORE) {
        auto epi = [&](int row, int bi, float v) {
            if (bi >= a.nb) return;
            if (a.relu) v = fmaxf(v, 0.f);
            a.y[size_t(bi) * a.w.N + row] = v;
        };
        gemv_rows<T, B, CPL, false, 1>(a.w, a.g, xr, gwave, nwaves, pre, prologue, epi, a.bias);
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
        gemv_rows<T, B, CPL, false, 1>(a.w, a.g, xr, gwave, nwaves, pre, prologue, epi, a.bias);
    }
}

// ------------------------------------------------------------------ attn_head

struct HeadArgs {
    WPtr w;          // out-projection [d][d]
    int nb, d, H, L;
    int HG;          // heads per workgroup (C = HG * HD columns of W)
    int RW;          // rows of W per workgroup
    const float *q;  // [nb][d]
    const __half *K, *V;   // [nb][H][L][HD]
    const uint32_t *lens;  // cross lengths, or null: *step + 1 keys
    const uint32_t *step;
    float *part;     // [H / HG][nb][d]
    const uint32_t *rows;  // optional [nb][L]: cache row holding slot j of row bi (beam search)
};

constexpr int kHeadCols = 256;  // max columns (HG * HD) per workgroup
constexpr int kHeadParts = 8;   // head groups are sized so that P = H / HG <= this when possible

// ---- one (row, head) pair shared by two waves (batch 1, head groups of <= 2 heads) ----
// Wave q of the pair takes the SPL-key groups 2 i + q: pass u of its chunk c covers keys
// SPL (2 (c U2 + u) + q) + split.  Each wave keeps an online softmax over its keys and
// leaves its partial in LDS: po[HD] = sum_j p_j v_j (unnormalized), pml = (max, sum_j p_j)
// with p_j = exp(s_j - max).  attn_combine2 then rescales the two partials to their common
// max and divides: the same keys and the same order of sums whichever kernel runs it.
constexpr int kHalfU = 4;                  // passes per chunk of a half
constexpr int kHalfSlot = 128 + 2;         // floats of one wave's partial (HD <= 128)
__host__ __device__ constexpr int half_key(int spl, int c, int u, int q) { return spl * (2 * (c * kHalfU + u) + q); }

template <int HD, class LoadF>
__device__ __forceinline__ void attn_half(int n, int q, const float4 &qa, const float4 &qb, const uint4 (&kr)[kHalfU],
                                          const uint4 (&vr)[kHalfU], LoadF &&load, float *wsc, float *slot) {
    constexpr int TPK = HD / 8, SPL = 64 / TPK;
    const int lane = threadIdx.x & 63, sub = lane % TPK, split = lane / TPK;
    float m = -INFINITY, l = 0.f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int c = 0; half_key(SPL, c, 0, q) < n; ++c) {  // wave-uniform; chunk 0 is in flight
        if (c) load(c);
        float sc[kHalfU];
        float cmax = -INFINITY;
#pragma unroll
        for (int u = 0; u < kHalfU; ++u) {
            float s = h2f(kr[u].x) * qa.x;
            s = fmaf(h2f(kr[u].x >> 16), qa.y, s);
            s = fmaf(h2f(kr[u].y), qa.z, s);
            s = fmaf(h2f(kr[u].y >> 16), qa.w, s);
            s = fmaf(h2f(kr[u].z), qb.x, s);
            s = fmaf(h2f(kr[u].z >> 16), qb.y, s);
            s = fmaf(h2f(kr[u].w), qb.z, s);
            s = fmaf(h2f(kr[u].w >> 16), qb.w, s);
            s = group_sum<TPK>(s);
            sc[u] = half_key(SPL, c, u, q) + split < n ? s : -INFINITY;
            cmax = fmaxf(cmax, sc[u]);
        }
        const float mnew = fmaxf(m, wave_max(cmax));  // finite: the chunk's first key is valid
        const float r = expf(m - mnew);
        l *= r;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= r;
#pragma unroll
        for (int u = 0; u < kHalfU; ++u) {
            const bool in = half_key(SPL, c, u, q) + split < n;
            const float pj = in ? expf(sc[u] - mnew) : 0.f;
            l += pj;
            const uint32_t wv[4] = {in ? vr[u].x : 0u, in ? vr[u].y : 0u, in ? vr[u].z : 0u, in ? vr[u].w : 0u};
#pragma unroll
            for (int q2 = 0; q2 < 4; ++q2) {
                acc[2 * q2] = fmaf(pj, h2f(wv[q2]), acc[2 * q2]);
                acc[2 * q2 + 1] = fmaf(pj, h2f(wv[q2] >> 16), acc[2 * q2 + 1]);
            }
        }
        m = mnew;
    }
    // every lane of a split holds that split's sum; count each split once
    const float lsum = wave_sum(sub == 0 ? l : 0.f);
#pragma unroll
    for (int e = 0; e < 8; ++e) wsc[lane * 8 + e] = acc[e];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    for (int e = lane; e < HD; e += 64) {
        float o = 0.f;
#pragma unroll
        for (int s2 = 0; s2 < SPL; ++s2) o += wsc[(s2 * TPK + e / 8) * 8 + e % 8];
        slot[e] = o;
    }
    if (lane == 0) {
        slot[HD] = m;  // -inf when this wave had no key
        slot[HD + 1] = lsum;
    }
}

// out[e] of the pair from the partials of its two waves (after a workgroup barrier)
template <int HD>
__device__ __forceinline__ void attn_combine2(const float *s0, const float *s1, float *out) {
    const int lane = threadIdx.x & 63;
    const float m0 = s0[HD], m1 = s1[HD], M = fmaxf(m0, m1);  // m0 finite: wave 0 has key 0
    const float e0 = expf(m0 - M), e1 = expf(m1 - M);
    const float inv = 1.f / (e0 * s0[HD + 1] + e1 * s1[HD + 1]);
    for (int e = lane; e < HD; e += 64) out[e] = (e0 * s0[e] + e1 * s1[e]) * inv;
}

// Workgroup (g, r): attention of heads [g HG, (g + 1) HG) for all nb rows, then
// part[g][bi][row] = sum_{c < C} W[row][g C + c] * att[bi][g C + c] for the RW
// rows [r RW, (r + 1) RW), one (row, chunk) item per thread.  Workgroups with the
// same g repeat the attention (a few KB of K/V from L2) so that the projection
// is spread over many CUs.
//
// Attention runs one (row, head) pair per wave with no workgroup barrier: lane
// (split, sub) owns dimensions [8 sub, 8 sub + 8) of the keys j = k SPL + split,
// so the score a lane computes (summed over the TPK lanes of its split) is the
// weight it applies to its own values.  Keys are consumed in chunks of U SPL with
// an online softmax (running max and sum), so any length fits in registers.
// S2 (batch 1, head groups of <= 2 heads): two waves per pair (attn_half).
template <int T, int HD, bool S2>
__global__ __launch_bounds__(256) void k_attn_head(HeadArgs a) {
    constexpr int XW = GTraits<T>::XW, NS = GTraits<T>::NS;
    constexpr int TPK = HD / 8;     // lanes per key: 8-wide dimension groups
    constexpr int SPL = 64 / TPK;   // keys per pass of a wave
    constexpr int U = 8;            // passes per chunk (loads in flight)
    extern __shared__ float lds[];
    // w a scalar: branches on it stay uniform (no divergent load paths)
    const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int nb = a.nb, d = a.d, H = a.H, L = a.L, HG = a.HG, hg_log2 = __builtin_ctz(a.HG);
    const int C = HG * HD, g = blockIdx.x, h0 = g * HG, col0 = g * C;
    const int pairs = nb * HG;
    float *outv = lds;                           // [pairs][HD] = [nb][C]
    float *wsc = lds + 4 * kHeadCols + w * 512;  // this wave's [64][8] scratch
    float *slots = lds + 4 * kHeadCols + 4 * 512;  // S2: [4 waves][kHalfSlot]
    const int sub = lane % TPK, split = lane / TPK;

    // Order of issue: the first chunk of this wave's first pair (addresses do not
    // depend on the key counts; keys past a row's count are masked when used),
    // the projection's weights, then the key counts.  Loads complete in order, so
    // the attention never waits for the weights.
    uint4 kr[U], vr[U];
    float4 qa, qb;
    auto load_chunk_kv = [&](int p, int j0) {
        const int bi = p >> hg_log2, hh = h0 + (p & (HG - 1));
        // the cache rows first (beam search's row map; greedy: the row itself), then every
        // K/V load back to back (a row lookup per key would make each pair wait for the last)
        uint32_t r[U];
        if (a.rows) {  // kernel argument
#pragma unroll
            for (int u = 0; u < U; ++u) r[u] = a.rows[size_t(bi) * L + min(j0 + u * SPL + split, L - 1)];
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) r[u] = uint32_t(bi);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = min(j0 + u * SPL + split, L - 1);
            const size_t o = ((size_t(r[u]) * H + hh) * L + j) * HD + sub * 8;
            kr[u] = *reinterpret_cast<const uint4 *>(a.K + o);
            vr[u] = *reinterpret_cast<const uint4 *>(a.V + o);
        }
        const float *qp = a.q + size_t(bi) * d + hh * HD + sub * 8;
        qa = *reinterpret_cast<const float4 *>(qp);
        qb = *reinterpret_cast<const float4 *>(qp + 4);
    };
    // S2: chunk c of wave q of pair p (rows first, as above)
    uint4 kr2[kHalfU], vr2[kHalfU];
    auto load_half = [&](int p, int q, int c) {
        const int hh = h0 + p;
        uint32_t r[kHalfU];
        if (a.rows) {  // kernel argument
#pragma unroll
            for (int u = 0; u < kHalfU; ++u) r[u] = a.rows[min(half_key(SPL, c, u, q) + split, L - 1)];
        } else {
#pragma unroll
            for (int u = 0; u < kHalfU; ++u) r[u] = 0u;
        }
#pragma unroll
        for (int u = 0; u < kHalfU; ++u) {
            const int j = min(half_key(SPL, c, u, q) + split, L - 1);
            const size_t o = ((size_t(r[u]) * H + hh) * L + j) * HD + sub * 8;
            kr2[u] = *reinterpret_cast<const uint4 *>(a.K + o);
            vr2[u] = *reinterpret_cast<const uint4 *>(a.V + o);
        }
        if (c == 0) {
            const float *qp = a.q + hh * HD + sub * 8;
            qa = *reinterpret_cast<const float4 *>(qp);
            qb = *reinterpret_cast<const float4 *>(qp + 4);
        }
    };
    if constexpr (S2) {
        if (w < 2 * pairs) load_half(w >> 1, w & 1, 0);
    } else {
        if (w < pairs) load_chunk_kv(w, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    const int CPR = C / XW, cpr_log2 = __builtin_ctz(CPR), c0 = col0 / XW;
    const int rl = t >> cpr_log2, wcc = t & (CPR - 1);
    const int wrow = blockIdx.y * a.RW + rl;
    const bool wok = rl < a.RW && wrow < d;
    Raw<T> wr;
    load_chunk<T>(a.w, wok ? wrow : blockIdx.y * a.RW, c0 + wcc, wr);
    __builtin_amdgcn_sched_barrier(0);

    // key counts per row: wave-uniform (scalar) loads
    const int n_self = a.lens ? 0 : int(*a.step) + 1;
    int nk[4];
#pragma unroll
    for (int bi = 0; bi < 4; ++bi) nk[bi] = bi < nb ? (a.lens ? int(a.lens[bi]) : n_self) : 0;

    if constexpr (S2) {
        if (w < 2 * pairs)
            attn_half<HD>(nk[0], w & 1, qa, qb, kr2, vr2, [&](int c) { load_half(w >> 1, w & 1, c); }, wsc,
                          slots + w * kHalfSlot);
        lds_barrier();
        if (w < pairs) attn_combine2<HD>(slots + 2 * w * kHalfSlot, slots + (2 * w + 1) * kHalfSlot, outv + w * HD);
    } else {
        for (int p = w; p < pairs; p += 4) {  // wave-uniform
            const int bi = p >> hg_log2;
            const int n = bi == 0 ? nk[0] : bi == 1 ? nk[1] : bi == 2 ? nk[2] : nk[3];
            float m = -INFINITY, l = 0.f;
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int j0 = 0; j0 < n; j0 += U * SPL) {
                if (p != w || j0 != 0) load_chunk_kv(p, j0);
                float sc[U];
                float cmax = -INFINITY;
    #pragma unroll
                for (int u = 0; u < U; ++u) {
                    float s = h2f(kr[u].x) * qa.x;
                    s = fmaf(h2f(kr[u].x >> 16), qa.y, s);
                    s = fmaf(h2f(kr[u].y), qa.z, s);
                    s = fmaf(h2f(kr[u].y >> 16), qa.w, s);
                    s = fmaf(h2f(kr[u].z), qb.x, s);
                    s = fmaf(h2f(kr[u].z >> 16), qb.y, s);
                    s = fmaf(h2f(kr[u].w), qb.z, s);
                    s = fmaf(h2f(kr[u].w >> 16), qb.w, s);
                    s = group_sum<TPK>(s);
                    sc[u] = j0 + u * SPL + split < n ? s : -INFINITY;
                    cmax = fmaxf(cmax, sc[u]);
                }
                const float mnew = fmaxf(m, wave_max(cmax));  // finite: key j0 is valid
                const float r = expf(m - mnew);
                l *= r;
    #pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] *= r;
    #pragma unroll
                for (int u = 0; u < U; ++u) {
                    const bool in = j0 + u * SPL + split < n;
                    const float pj = in ? expf(sc[u] - mnew) : 0.f;
                    l += pj;
                    const uint32_t wv[4] = {in ? vr[u].x : 0u, in ? vr[u].y : 0u, in ? vr[u].z : 0u, in ? vr[u].w : 0u};
    #pragma unroll
                    for (int q2 = 0; q2 < 4; ++q2) {
                        acc[2 * q2] = fmaf(pj, h2f(wv[q2]), acc[2 * q2]);
                        acc[2 * q2 + 1] = fmaf(pj, h2f(wv[q2] >> 16), acc[2 * q2 + 1]);
                    }
                }
                m = mnew;
            }
            // every lane of a split holds that split's sum; count each split once
            const float inv = 1.f / wave_sum(sub == 0 ? l : 0.f);
    #pragma unroll
            for (int e = 0; e < 8; ++e) wsc[lane * 8 + e] = acc[e];
            __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS writes are done
            __builtin_amdgcn_wave_barrier();
            for (int e = lane; e < HD; e += 64) {
                float o = 0.f;
    #pragma unroll
                for (int s2 = 0; s2 < SPL; ++s2) o += wsc[(s2 * TPK + e / 8) * 8 + e % 8];
                outv[p * HD + e] = o * inv;
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
        }
    }
    lds_barrier();

    // the group's slice of the out-projection
    const int c = c0 + wcc;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int bi = 0; bi < 4; ++bi) {
        if (bi >= nb) break;
        XF<T, 1> X;
#pragma unroll
        for (int e = 0; e < XW; e += 4) {
            const float4 x4 = *reinterpret_cast<const float4 *>(outv + bi * C + xpos<T>(c, e) - col0);
            X.x[0][e] = x4.x;
            X.x[0][e + 1] = x4.y;
            X.x[0][e + 2] = x4.z;
            X.x[0][e + 3] = x4.w;
        }
#pragma unroll
        for (int s2 = 0; s2 < NS; ++s2) X.s[0][s2] = 0.f;
#pragma unroll
        for (int e = 0; e < XW; ++e) X.s[0][xslot<T>(e)] += X.x[0][e];
        float a1[1] = {0.f};
        dot_chunk<T, 1>(c, wr, X, a1);
        acc[bi] = a1[0];
    }
#pragma unroll
    for (int bi = 0; bi < 4; ++bi) acc[bi] = group_sum_dyn(acc[bi], cpr_log2);
    if (wcc == 0 && wok)
        for (int bi = 0; bi < nb; ++bi) a.part[(size_t(g) * nb + bi) * d + wrow] = acc[bi];
}

// ------------------------------------------- cross attention with its q projection

constexpr int kXThreads = 512;  // 8 waves
constexpr int kXItems = 4;      // (row, chunk) items of the q projection per thread

// dot4u8 as one asm block: each byte is converted where it is used, so a schedule
// cannot convert every item's bytes ahead of their products (which overflows the
// registers of a multi-item dot); same operations, same order
[[maybe_unused]] __device__ __forceinline__ float dot4u8_chain(uint32_t v, const float (&x)[4], float acc) {
    float t0, t1, t2, t3;
    asm("v_cvt_f32_ubyte0 %1, %5\n\t"
        "v_cvt_f32_ubyte1 %2, %5\n\t"
        "v_fmac_f32 %0, %1, %6\n\t"
        "v_cvt_f32_ubyte2 %3, %5\n\t"
        "v_fmac_f32 %0, %2, %7\n\t"
        "v_cvt_f32_ubyte3 %4, %5\n\t"
        "v_fmac_f32 %0, %3, %8\n\t"
        "v_fmac_f32 %0, %4, %9"
        : "+v"(acc), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
        : "v"(v), "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]));
    return acc;
}

// dot4u8_chain of four items' words against the same four x values, as one asm block:
// byte b of every word is converted, then the four products are added, so the four
// items' dependent chains interleave (one chain per block left each product waiting for
// the previous one); per item the operations and their order are dot4u8_chain's
__device__ __forceinline__ void dot4u8_chain4(const uint32_t (&v)[4], const float (&x)[4], float (&acc)[4]) {
    float t0, t1, t2, t3;
    asm("v_cvt_f32_ubyte0 %4, %8\n\t"
        "v_cvt_f32_ubyte0 %5, %9\n\t"
        "v_cvt_f32_ubyte0 %6, %10\n\t"
        "v_cvt_f32_ubyte0 %7, %11\n\t"
        "v_fmac_f32 %0, %4, %12\n\t"
        "v_fmac_f32 %1, %5, %12\n\t"
        "v_fmac_f32 %2, %6, %12\n\t"
        "v_fmac_f32 %3, %7, %12\n\t"
        "v_cvt_f32_ubyte1 %4, %8\n\t"
        "v_cvt_f32_ubyte1 %5, %9\n\t"
        "v_cvt_f32_ubyte1 %6, %10\n\t"
        "v_cvt_f32_ubyte1 %7, %11\n\t"
        "v_fmac_f32 %0, %4, %13\n\t"
        "v_fmac_f32 %1, %5, %13\n\t"
        "v_fmac_f32 %2, %6, %13\n\t"
        "v_fmac_f32 %3, %7, %13\n\t"
        "v_cvt_f32_ubyte2 %4, %8\n\t"
        "v_cvt_f32_ubyte2 %5, %9\n\t"
        "v_cvt_f32_ubyte2 %6, %10\n\t"
        "v_cvt_f32_ubyte2 %7, %11\n\t"
        "v_fmac_f32 %0, %4, %14\n\t"
        "v_fmac_f32 %1, %5, %14\n\t"
        "v_fmac_f32 %2, %6, %14\n\t"
        "v_fmac_f32 %3, %7, %14\n\t"
        "v_cvt_f32_ubyte3 %4, %8\n\t"
        "v_cvt_f32_ubyte3 %5, %9\n\t"
        "v_cvt_f32_ubyte3 %6, %10\n\t"
        "v_cvt_f32_ubyte3 %7, %11\n\t"
        "v_fmac_f32 %0, %4, %15\n\t"
        "v_fmac_f32 %1, %5, %15\n\t"
        "v_fmac_f32 %2, %6, %15\n\t"
        "v_fmac_f32 %3, %7, %15"
        : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
        : "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]));
}

// group_sum_dyn of N values at once, step by step, so that their DPP chains interleave
// (per value the same operations in the same order)
template <int N>
__device__ __forceinline__ void group_sum_dyn_n(float (&v)[N], int log2w) {
    if (log2w >= 1)
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = v[i] + dpp_mov<kDppXor1>(v[i]);
    if (log2w >= 2)
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = v[i] + dpp_mov<kDppXor2>(v[i]);
    if (log2w >= 3)
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = v[i] + dpp_mov<kDppHalfMirror>(v[i]);
    if (log2w >= 4)
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = v[i] + dpp_mov<kDppMirror>(v[i]);
    if (log2w >= 5)
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const float r0 = lane_value(v[i], 0), r1 = lane_value(v[i], 16), r2 = lane_value(v[i], 32),
                        r3 = lane_value(v[i], 48);
            v[i] = log2w == 5 ? ((threadIdx.x & 32) ? r2 + r3 : r0 + r1) : (r0 + r1) + (r2 + r3);
        }
}

// dot_chunk of KI q4_K / q5_K items that share chunk c, with x read from LDS (xc:
// the chunk's 64 contiguous values) one float4 at a time and applied to every item,
// so no item's values are expanded all at once.  Per item the operations and their
// order are those of dot_chunk with f32 x (one row): the results are equal.
template <int T, int KI>
__device__ __forceinline__ void dot_items(int c, const Raw<T> (&r)[KI], const float *xc, float (&out)[KI]) {
    static_assert(T == GGML_Q4_K || T == GGML_Q5_K, "q4_K / q5_K only");
    const int g = c & 3;
    float al[KI], ah[KI];
#pragma unroll
    for (int k = 0; k < KI; ++k) al[k] = ah[k] = 0.f;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const float4 xl = *reinterpret_cast<const float4 *>(xc + 4 * u);
        const float4 xh = *reinterpret_cast<const float4 *>(xc + 32 + 4 * u);
        const float vl[4] = {xl.x, xl.y, xl.z, xl.w}, vh[4] = {xh.x, xh.y, xh.z, xh.w};
        uint32_t lo[KI], hi[KI];
#pragma unroll
        for (int k = 0; k < KI; ++k) {
            const uint32_t wu = u < 4 ? (&r[k].a.x)[u] : (&r[k].b.x)[u - 4];
            if constexpr (T == GGML_Q5_K) {
                const uint32_t hb = u < 4 ? (&r[k].c.x)[u] : (&r[k].e.x)[u - 4];
                lo[k] = (wu & 0x0F0F0F0Fu) | (((hb >> (2 * g)) & 0x01010101u) << 4);
                hi[k] = ((wu >> 4) & 0x0F0F0F0Fu) | (((hb >> (2 * g + 1)) & 0x01010101u) << 4);
            } else {
                lo[k] = wu & 0x0F0F0F0Fu;
                hi[k] = wu & 0xF0F0F0F0u;  // 16 * nibble; scaled back below
            }
        }
        if constexpr (KI == 4) {
            dot4u8_chain4(lo, vl, al);
            dot4u8_chain4(hi, vh, ah);
        } else {
#pragma unroll
            for (int k = 0; k < KI; ++k) {
                al[k] = dot4u8_chain(lo[k], vl, al[k]);
                ah[k] = dot4u8_chain(hi[k], vh, ah[k]);
            }
        }
    }
    // the sums of gemv_load_x (xslot: values 0..31 -> 0, 32..63 -> 1), in its order
#pragma unroll
    for (int e = 0; e < 32; ++e) s0 += xc[e];
#pragma unroll
    for (int e = 32; e < 64; ++e) s1 += xc[e];
    const int sh0 = 8 * ((2 * g) & 3), sh1 = sh0 + 8;
    const bool upper = g >= 2;
#pragma unroll
    for (int k = 0; k < KI; ++k) {
        auto decode = [&](int sh, float &sc, float &mn) {
            const uint32_t B0 = r[k].h.y >> sh, B1 = r[k].h.z >> sh, B2 = r[k].h.w >> sh;
            const uint32_t a = upper ? ((B2 & 15u) | ((B0 >> 2) & 48u)) : (B0 & 63u);
            const uint32_t bb = upper ? (((B2 >> 4) & 15u) | ((B1 >> 2) & 48u)) : (B1 & 63u);
            sc = float(a);
            mn = float(bb);
        };
        float sc0, m0, sc1, m1;
        decode(sh0, sc0, m0);
        decode(sh1, sc1, m1);
        const float d = h2f(r[k].h.x), dmin = h2f(r[k].h.x >> 16);
        float a0 = ah[k];
        if constexpr (T == GGML_Q4_K) a0 *= 0.0625f;
        float acc = 0.f;
        acc += d * (sc0 * al[k] + sc1 * a0) - dmin * (m0 * s0 + m1 * s1);
        out[k] = acc;
    }
}

struct XAttnArgs {
    StepArgs s;            // residual prologue: x_in + self-attention partials + b_out, cross_norm
    WPtr wq;               // cross_q [d][d]
    const float *bq;
    WPtr wo;               // cross_out [d][d]
    int H, L, HG, RW;
    const __half *K, *V;   // cross K/V [nb][H][L][HD]
    const uint32_t *lens;  // [nb]
    float *part;           // out: [H / HG][nb][d] (another buffer than s.part)
};

// cross_q, the cross attention and its out-projection slice in one launch (PR = batch
// rows <= 2, d <= 1024, at most kPreParts self-attention partials).  Workgroup (g, r) rebuilds x = x_in + sum of the self-attention
// partials + b_out (workgroup (0, 0) stores it), applies cross_norm, computes q for
// heads [g HG, (g + 1) HG) from the C rows of Wq it needs (at most kXItems (row, chunk)
// items per thread, all issued at entry with the out-projection's weights), then
// runs the attention and projection of k_attn_head.  The workgroups of one group
// repeat those C rows (72 KB at 600M, from L2) instead of waiting for a separate
// launch.  Every sum is in the order of the separate kernels, so the partials equal
// theirs bit for bit.
// S2 (batch 1, head groups of <= 2 heads): two waves per pair (attn_half), as k_attn_head.
template <int T, int HD, int PR, bool S2>
__global__ __launch_bounds__(kXThreads) void k_xattn(XAttnArgs a) {
    constexpr int XW = GTraits<T>::XW, NS = GTraits<T>::NS;
    constexpr int TPK = HD / 8, SPL = 64 / TPK, U = 8, NW = kXThreads / 64;
    extern __shared__ float lds[];
    __shared__ double red[2 * 4 * NW];
    // w a scalar: branches on it stay uniform (no divergent load paths)
    const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int nb = a.s.nb, d = a.s.d, H = a.H, L = a.L, HG = a.HG, hg_log2 = __builtin_ctz(a.HG);
    const int C = HG * HD, g = blockIdx.x, h0 = g * HG, col0 = g * C;
    const int pairs = nb * HG;
    const int ldx = lds_pad(d);
    float *xs = lds;                // [nb][ldx]: cross_norm(x)
    float *qs = xs + nb * ldx;      // [nb][C]
    float *outv = qs + nb * C;      // [nb][C] = [pairs][HD]
    float *wsc = outv + nb * C + w * 512;  // attention waves: [64][8] scratch
    float *slots = outv + nb * C + 4 * 512;  // S2: [4 waves][kHalfSlot]

    // Order of issue: residual operands (the prologue waits for them first), the q
    // rows, the out-projection chunk, the first K/V chunk.  Loads complete in order,
    // so each phase waits only for what it uses.
    PreLoadsR<PR> PL;
    if (w < 4) {  // scalar: the threads that own the float4 slots
        preload<PR>(a.s, PL);
    } else {
#pragma unroll
        for (int bi = 0; bi < PR; ++bi) {
#pragma unroll
            for (int p = 0; p < kPreParts; ++p) PL.part[bi][p] = make_float4(0.f, 0.f, 0.f, 0.f);
            PL.x[bi] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        PL.pb = PL.gr = PL.br = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int CQ = a.wq.K / XW, cq_log2 = __builtin_ctz(CQ), qc = t & (CQ - 1);
    Raw<T> wq[kXItems];
    float qbias[kXItems];
#pragma unroll
    for (int k = 0; k < kXItems; ++k) {
        const int row = (t + k * kXThreads) >> cq_log2;
        const int r = col0 + (row < C ? row : 0);
        load_chunk<T>(a.wq, r, qc, wq[k]);
        qbias[k] = a.bq[r];
    }
    const int CPR = C / XW, cpr_log2 = __builtin_ctz(CPR), c0 = col0 / XW;
    const int rl = t >> cpr_log2, wcc = t & (CPR - 1);
    const int wrow = blockIdx.y * a.RW + rl;
    const bool wok = rl < a.RW && wrow < d;
    Raw<T> wr;
    load_chunk<T>(a.wo, wok ? wrow : 0, c0 + wcc, wr);
    // batch 1: the first key chunk of this wave's first (row, head) pair (addresses
    // do not depend on the key counts; keys past a row's count are masked when used)
    const int sub = lane % TPK, split = lane / TPK;
    uint4 kr[U], vr[U];
    auto load_kv = [&](int p, int j0) {
        const int bi = p >> hg_log2, hh = h0 + (p & (HG - 1));
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = min(j0 + u * SPL + split, L - 1);
            const size_t o = ((size_t(bi) * H + hh) * L + j) * HD + sub * 8;
            kr[u] = *reinterpret_cast<const uint4 *>(a.K + o);
            vr[u] = *reinterpret_cast<const uint4 *>(a.V + o);
        }
    };
    // S2: chunk c of wave q of head p (batch 1)
    uint4 kr2[kHalfU], vr2[kHalfU];
    auto load_half = [&](int p, int q, int c) {
        const int hh = h0 + p;
#pragma unroll
        for (int u = 0; u < kHalfU; ++u) {
            const int j = min(half_key(SPL, c, u, q) + split, L - 1);
            const size_t o = (size_t(hh) * L + j) * HD + sub * 8;
            kr2[u] = *reinterpret_cast<const uint4 *>(a.K + o);
            vr2[u] = *reinterpret_cast<const uint4 *>(a.V + o);
        }
    };
    constexpr bool kEarlyKV = PR == 1;  // two rows' q would not fit the registers beside them
    if constexpr (S2) {
        if (w < 2 * pairs) load_half(w >> 1, w & 1, 0);
    } else {
        if (kEarlyKV && w < pairs) load_kv(w, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    int nk[PR];
#pragma unroll
    for (int bi = 0; bi < PR; ++bi) nk[bi] = bi < nb ? int(a.lens[bi]) : 0;

    resid_ln_prologue<PRO_RESID_PRE, GGML_F32, NW, 1, PR>(a.s, PL, xs, red);

    // q = cross_norm(x) Wq^T + bq for this group's C rows, as k_step computes them
    {
        float acc[kXItems][PR];
#pragma unroll
        for (int bi = 0; bi < PR; ++bi) {
#pragma unroll
            for (int k = 0; k < kXItems; ++k) acc[k][bi] = 0.f;
            if (bi >= nb) continue;
            float o[kXItems];
            dot_items<T, kXItems>(qc, wq, xs + bi * ldx + lds_pad(xpos<T>(qc, 0)), o);
#pragma unroll
            for (int k = 0; k < kXItems; ++k) acc[k][bi] = o[k];
        }
        float sums[kXItems * PR];
#pragma unroll
        for (int k = 0; k < kXItems; ++k)
#pragma unroll
            for (int bi = 0; bi < PR; ++bi) sums[k * PR + bi] = acc[k][bi];
        group_sum_dyn_n(sums, cq_log2);
#pragma unroll
        for (int k = 0; k < kXItems; ++k) {
            const int row = (t + k * kXThreads) >> cq_log2;
#pragma unroll
            for (int bi = 0; bi < PR; ++bi)
                if (qc == 0 && row < C && bi < nb) qs[bi * C + row] = sums[k * PR + bi] + qbias[k];
        }
    }
    lds_barrier();

    if constexpr (S2) {
        if (w < 2 * pairs) {
            const float4 qa = *reinterpret_cast<const float4 *>(qs + (w >> 1) * HD + sub * 8);
            const float4 qb = *reinterpret_cast<const float4 *>(qs + (w >> 1) * HD + sub * 8 + 4);
            attn_half<HD>(nk[0], w & 1, qa, qb, kr2, vr2, [&](int c) { load_half(w >> 1, w & 1, c); }, wsc,
                          slots + w * kHalfSlot);
        }
        lds_barrier();
        if (w < pairs) attn_combine2<HD>(slots + 2 * w * kHalfSlot, slots + (2 * w + 1) * kHalfSlot, outv + w * HD);
    } else {
        // attention: one (row, head) pair per wave, as in k_attn_head
        for (int p = w; p < pairs; p += NW) {  // wave-uniform
            const int bi = p >> hg_log2, hl = p & (HG - 1);
            const int n = PR == 1 || bi == 0 ? nk[0] : nk[PR - 1];
            const float4 qa = *reinterpret_cast<const float4 *>(qs + bi * C + hl * HD + sub * 8);
            const float4 qb = *reinterpret_cast<const float4 *>(qs + bi * C + hl * HD + sub * 8 + 4);
            float m = -INFINITY, l = 0.f;
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int j0 = 0; j0 < n; j0 += U * SPL) {
                if (!kEarlyKV || p != w || j0 != 0) load_kv(p, j0);
                float sc[U];
                float cmax = -INFINITY;
    #pragma unroll
                for (int u = 0; u < U; ++u) {
                    float s = h2f(kr[u].x) * qa.x;
                    s = fmaf(h2f(kr[u].x >> 16), qa.y, s);
                    s = fmaf(h2f(kr[u].y), qa.z, s);
                    s = fmaf(h2f(kr[u].y >> 16), qa.w, s);
                    s = fmaf(h2f(kr[u].z), qb.x, s);
                    s = fmaf(h2f(kr[u].z >> 16), qb.y, s);
                    s = fmaf(h2f(kr[u].w), qb.z, s);
                    s = fmaf(h2f(kr[u].w >> 16), qb.w, s);
                    s = group_sum<TPK>(s);
                    sc[u] = j0 + u * SPL + split < n ? s : -INFINITY;
                    cmax = fmaxf(cmax, sc[u]);
                }
                const float mnew = fmaxf(m, wave_max(cmax));
                const float r = expf(m - mnew);
                l *= r;
    #pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] *= r;
    #pragma unroll
                for (int u = 0; u < U; ++u) {
                    const bool in = j0 + u * SPL + split < n;
                    const float pj = in ? expf(sc[u] - mnew) : 0.f;
                    l += pj;
                    const uint32_t wv[4] = {in ? vr[u].x : 0u, in ? vr[u].y : 0u, in ? vr[u].z : 0u, in ? vr[u].w : 0u};
    #pragma unroll
                    for (int q2 = 0; q2 < 4; ++q2) {
                        acc[2 * q2] = fmaf(pj, h2f(wv[q2]), acc[2 * q2]);
                        acc[2 * q2 + 1] = fmaf(pj, h2f(wv[q2] >> 16), acc[2 * q2 + 1]);
                    }
                }
                m = mnew;
            }
            const float inv = 1.f / wave_sum(sub == 0 ? l : 0.f);
    #pragma unroll
            for (int e = 0; e < 8; ++e) wsc[lane * 8 + e] = acc[e];
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
            for (int e = lane; e < HD; e += 64) {
                float o = 0.f;
    #pragma unroll
                for (int s2 = 0; s2 < SPL; ++s2) o += wsc[(s2 * TPK + e / 8) * 8 + e % 8];
                outv[p * HD + e] = o * inv;
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
        }
    }
    lds_barrier();

    // the group's slice of the out-projection
    const int c = c0 + wcc;
    float acc[PR];
#pragma unroll
    for (int bi = 0; bi < PR; ++bi) {
        acc[bi] = 0.f;
        if (bi >= nb) break;
        XF<T, 1> X;
#pragma unroll
        for (int e = 0; e < XW; e += 4) {
            const float4 x4 = *reinterpret_cast<const float4 *>(outv + bi * C + xpos<T>(c, e) - col0);
            X.x[0][e] = x4.x;
            X.x[0][e + 1] = x4.y;
            X.x[0][e + 2] = x4.z;
            X.x[0][e + 3] = x4.w;
        }
#pragma unroll
        for (int s2 = 0; s2 < NS; ++s2) X.s[0][s2] = 0.f;
#pragma unroll
        for (int e = 0; e < XW; ++e) X.s[0][xslot<T>(e)] += X.x[0][e];
        float a1[1] = {0.f};
        dot_chunk<T, 1>(c, wr, X, a1);
        acc[bi] = a1[0];
    }
#pragma unroll
    for (int bi = 0; bi < PR; ++bi) acc[bi] = group_sum_dyn(acc[bi], cpr_log2);
    if (wcc == 0 && wok)
#pragma unroll
        for (int bi = 0; bi < PR; ++bi)
            if (bi < nb) a.part[(size_t(g) * nb + bi) * d + wrow] = acc[bi];
}

// ---------------------------------------------------------------- dispatch

template <int T, int B, int CPL, int PRO, int EPI, int ET>
hipError_t launch_t(const StepArgs &a, int grid, size_t lds, hipStream_t st) {
    if constexpr (GTraits<T>::XW * B * CPL > kGemvMaxXRegs || (PRO == PRO_RESID_PRE && B > 2)) {
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

// The residual operands fit the registers of PreLoads.
bool preloadable(const StepArgs &a) { return a.nb <= 2 && a.d <= 1024 && a.P <= kPreParts; }

bool prepare(const DevMatrix &w, int nb, StepArgs &a, int *cpl) {
    if (nb < 1 || nb > 4 || nb > gemv_max_batch(w) || !gemv_geometry(w, &a.g, cpl)) return false;
    a.w = wptr_of(w);
    a.nb = nb;
    return true;
}

// columns of W one head group must cover: whole chunks, and for q6_K whole
// 128-column halves of a block (a chunk interleaves 16-value runs of a half)
int head_unit(uint32_t type) { return type == GGML_Q6_K ? 128 : gemv_xw(type); }

struct HeadGeom {
    int HG, P, RW, R;
    size_t lds;
};

bool head_geometry(const DevMatrix &w, int nb, int d, int H, int hd, int L, HeadGeom *hg) {
    const int xw = gemv_xw(w.type), unit = head_unit(w.type);
    if (!xw || nb < 1 || nb > 4 || H < 1 || hd * H != d || w.N != d || w.K != d || L < 1) return false;
    if (hd != 16 && hd != 64 && hd != 128) return false;
    int HG = unit > hd ? unit / hd : 1;
    while (H / HG > kHeadParts && H % (2 * HG) == 0 && 2 * HG * hd <= kHeadCols) HG *= 2;
    const int C = HG * hd;
    if (C > kHeadCols || H % HG || C % xw || C % unit) return false;
    const int CPR = C / xw;  // a power of two
    if (CPR > 256) return false;
    const int RW = 256 / CPR < d ? 256 / CPR : d;
    hg->HG = HG;
    hg->P = H / HG;
    hg->RW = RW;
    hg->R = (d + RW - 1) / RW;
    hg->lds = sizeof(float) * (size_t(4) * kHeadCols + 4 * 512 + 4 * kHalfSlot);
    return true;
}

// two waves per (row, head) pair where the batch is one row and a group at most 2 heads
inline bool head_split2(int nb, int HG) { return nb == 1 && HG <= 2; }

template <int T, int HD>
hipError_t launch_head(const HeadArgs &a, int R, size_t lds, hipStream_t st) {
    if (head_split2(a.nb, a.HG))
        hipLaunchKernelGGL((k_attn_head<T, HD, true>), dim3(a.H / a.HG, R), dim3(256), lds, st, a);
    else
        hipLaunchKernelGGL((k_attn_head<T, HD, false>), dim3(a.H / a.HG, R), dim3(256), lds, st, a);
    return hipGetLastError();
}

template <int T>
hipError_t launch_head_hd(const HeadArgs &a, int hd, int R, size_t lds, hipStream_t st) {
    switch (hd) {
    case 16: return launch_head<T, 16>(a, R, lds, st);
    case 64: return launch_head<T, 64>(a, R, lds, st);
    case 128: return launch_head<T, 128>(a, R, lds, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool step_fusable(const DevMatrix &w, int nb, int d) {
    GemvGeom g;
    int cpl;
    if (nb < 1 || nb > 4 || nb > gemv_max_batch(w) || !gemv_geometry(w, &g, &cpl) || cpl > 2) return false;
    if (nb == 4 && cpl > 1) return false;
    // residual prologue: float4 slots, nb rows of d floats in LDS
    return d % 16 == 0 && d <= 1024 * kMaxF4 && size_t(nb) * lds_pad(d) * 4 + 512 <= 64 * 1024;
}

int step_head_parts(const DevMatrix &w, int nb, int d, int H, int hd, int L) {
    HeadGeom hg;
    return head_geometry(w, nb, d, H, hd, L, &hg) ? hg.P : 0;
}

bool step_embed_supported(uint32_t t, uint32_t e) {
    return (e == GGML_Q6_K && (t == GGML_Q4_K || t == GGML_Q5_K || t == GGML_Q6_K)) ||
           (t == e && (t == GGML_Q8_0 || t == GGML_F16 || t == GGML_F32));
}

hipError_t step_qkv(const DevMatrix &w, const float *bias, int nb, int d, const DevMatrix *emb, const uint32_t *ids,
                    const float *pos, uint32_t pos_base, float emb_scale, const float *x_in, const float *y_in,
                    float *x_out, const float *gamma, const float *beta, float eps, const uint32_t *step, float *q,
                    __half *kc, __half *vc, int H, int hd, int m, hipStream_t st, const SrcEmb &src) {
    StepArgs a{};
    int cpl;
    if (!prepare(w, nb, a, &cpl) || !step_fusable(w, nb, d) || w.N != 3 * d) return hipErrorInvalidValue;
    if (src.row && (!emb || !src.emb || src.S < 1)) return hipErrorInvalidValue;
    a.src_emb = src.emb;
    a.src_row = src.row;
    a.S = src.S;
    a.d = d;
    a.x_in = x_in;
    a.part = y_in;
    a.P = 1;
    a.x_out = x_out;
    a.gamma = gamma;
    a.beta = beta;
    a.eps = eps;
    if (emb) {
        a.eq = emb->q;
        a.es = emb->s;
        a.ed = emb->d;
        a.elast = uint32_t(emb->N - 1);
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
    const size_t lds = sizeof(float) * size_t(nb) * lds_pad(d);
    const int grid = gemv_grid(w, 1);
    const int B = gemv_round_b(nb);
    if (!emb)
        return preloadable(a) ? dispatch_t<PRO_RESID_PRE, EPI_QKV, GGML_F32>(w.type, a, B, cpl, grid, lds, st)
                              : dispatch_t<PRO_RESID, EPI_QKV, GGML_F32>(w.type, a, B, cpl, grid, lds, st);
    // (projection type, embedding type) pairs the presets produce (src/convert.rs:67-91)
    const uint32_t t = w.type, e = emb->type;
    if (t == GGML_Q4_K && e == GGML_Q6_K) return dispatch_bc<GGML_Q4_K, PRO_EMBED, EPI_QKV, GGML_Q6_K>(a, B, cpl, grid, lds, st);
    if (t == GGML_Q5_K && e == GGML_Q6_K) return dispatch_bc<GGML_Q5_K, PRO_EMBED, EPI_QKV, GGML_Q6_K>(a, B, cpl, grid, lds, st);
    if (t == GGML_Q6_K && e == GGML_Q6_K) return dispatch_bc<GGML_Q6_K, PRO_EMBED, EPI_QKV, GGML_Q6_K>(a, B, cpl, grid, lds, st);
    if (t == GGML_Q8_0 && e == GGML_Q8_0) return dispatch_bc<GGML_Q8_0, PRO_EMBED, EPI_QKV, GGML_Q8_0>(a, B, cpl, grid, lds, st);
    if (t == GGML_F16 && e == GGML_F16) return dispatch_bc<GGML_F16, PRO_EMBED, EPI_QKV, GGML_F16>(a, B, cpl, grid, lds, st);
    if (t == GGML_F32 && e == GGML_F32) return dispatch_bc<GGML_F32, PRO_EMBED, EPI_QKV, GGML_F32>(a, B, cpl, grid, lds, st);
    return hipErrorInvalidValue;
}

hipError_t step_attn_head(const DevMatrix &w, int nb, int d, const float *q, const __half *K, const __half *V, int H,
                          int hd, int L, const uint32_t *lens, const uint32_t *step, float *part, hipStream_t st,
                          const uint32_t *rows) {
    HeadGeom hg;
    if (!head_geometry(w, nb, d, H, hd, L, &hg)) return hipErrorInvalidValue;
    HeadArgs a{};
    a.w = wptr_of(w);
    a.nb = nb;
    a.d = d;
    a.H = H;
    a.L = L;
    a.HG = hg.HG;
    a.RW = hg.RW;
    a.q = q;
    a.K = K;
    a.V = V;
    a.lens = lens;
    a.step = step;
    a.part = part;
    a.rows = rows;
    switch (w.type) {
    case GGML_Q4_K: return launch_head_hd<GGML_Q4_K>(a, hd, hg.R, hg.lds, st);
    case GGML_Q5_K: return launch_head_hd<GGML_Q5_K>(a, hd, hg.R, hg.lds, st);
    case GGML_Q6_K: return launch_head_hd<GGML_Q6_K>(a, hd, hg.R, hg.lds, st);
    case GGML_Q8_0: return launch_head_hd<GGML_Q8_0>(a, hd, hg.R, hg.lds, st);
    case GGML_F16: return launch_head_hd<GGML_F16>(a, hd, hg.R, hg.lds, st);
    case GGML_F32: return launch_head_hd<GGML_F32>(a, hd, hg.R, hg.lds, st);
    default: return hipErrorInvalidValue;
    }
}

namespace {

template <int T, int HD>
hipError_t launch_xattn(const XAttnArgs &a, int R, size_t lds, hipStream_t st) {
    if (head_split2(a.s.nb, a.HG))
        hipLaunchKernelGGL((k_xattn<T, HD, 1, true>), dim3(a.H / a.HG, R), dim3(kXThreads), lds, st, a);
    else if (a.s.nb == 1)
        hipLaunchKernelGGL((k_xattn<T, HD, 1, false>), dim3(a.H / a.HG, R), dim3(kXThreads), lds, st, a);
    else
        hipLaunchKernelGGL((k_xattn<T, HD, 2, false>), dim3(a.H / a.HG, R), dim3(kXThreads), lds, st, a);
    return hipGetLastError();
}

template <int T>
hipError_t launch_xattn_hd(const XAttnArgs &a, int hd, int R, size_t lds, hipStream_t st) {
    switch (hd) {
    case 16: return launch_xattn<T, 16>(a, R, lds, st);
    case 64: return launch_xattn<T, 64>(a, R, lds, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool step_cross_fusable(const DevMatrix &wq, const DevMatrix &wo, int nb, int d, int H, int hd, int L, int P) {
    HeadGeom hg;
    if (P < 1 || P > kPreParts) return false;
    if (wq.type != wo.type || wq.N != d || wq.K != d || d > 1024 || d % 16 || nb < 1 || nb > 2) return false;
    if (hd != 16 && hd != 64) return false;
    if (wq.type != GGML_Q4_K && wq.type != GGML_Q5_K) return false;
    if (!head_geometry(wo, nb, d, H, hd, L, &hg)) return false;
    const int CQ = d / gemv_xw(wq.type), C = hg.HG * hd;
    // one lane group per q row (a power of two <= 64 lanes), at most kXItems items per thread
    return CQ >= 1 && CQ <= 64 && (CQ & (CQ - 1)) == 0 && size_t(C) * CQ <= size_t(kXItems) * kXThreads;
}

hipError_t step_cross_attn(const DevMatrix &wq, const float *bq, const DevMatrix &wo, int nb, int d, const float *x_in,
                           const float *part_in, int P, const float *pbias, float *x_out, const float *gamma,
                           const float *beta, float eps, const __half *K, const __half *V, int H, int hd, int L,
                           const uint32_t *lens, float *part_out, hipStream_t st) {
    HeadGeom hg;
    if (!step_cross_fusable(wq, wo, nb, d, H, hd, L, P) || part_in == part_out ||
        !head_geometry(wo, nb, d, H, hd, L, &hg))
        return hipErrorInvalidValue;
    XAttnArgs a{};
    a.s.nb = nb;
    a.s.d = d;
    a.s.x_in = x_in;
    a.s.part = part_in;
    a.s.P = P;
    a.s.pbias = pbias;
    a.s.x_out = x_out;
    a.s.gamma = gamma;
    a.s.beta = beta;
    a.s.eps = eps;
    a.wq = wptr_of(wq);
    a.bq = bq;
    a.wo = wptr_of(wo);
    a.H = H;
    a.L = L;
    a.HG = hg.HG;
    const int C = hg.HG * hd, CPR = C / gemv_xw(wo.type);
    a.RW = kXThreads / CPR < d ? kXThreads / CPR : d;
    const int R = (d + a.RW - 1) / a.RW;
    a.K = K;
    a.V = V;
    a.lens = lens;
    a.part = part_out;
    const int pairs = nb * hg.HG;
    // the attention waves' scratch (S2: 4 waves' and their partials)
    const size_t att = head_split2(nb, hg.HG) ? size_t(4) * 512 + 4 * kHalfSlot
                                              : size_t(pairs < kXThreads / 64 ? pairs : kXThreads / 64) * 512;
    const size_t lds = sizeof(float) * (size_t(nb) * lds_pad(d) + 2 * size_t(nb) * C + att);
    switch (wq.type) {
    case GGML_Q4_K: return launch_xattn_hd<GGML_Q4_K>(a, hd, R, lds, st);
    case GGML_Q5_K: return launch_xattn_hd<GGML_Q5_K>(a, hd, R, lds, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t step_resid_proj(const DevMatrix &w, const float *bias, bool relu, int nb, int d, const float *x_in,
                           const float *part, int P, const float *pbias, float *x_out, const float *gamma,
                           const float *beta, float eps, float *y, hipStream_t st) {
    StepArgs a{};
    int cpl;
    if (!prepare(w, nb, a, &cpl) || !step_fusable(w, nb, d) || P < 1 || w.K != d) return hipErrorInvalidValue;
    a.d = d;
    a.x_in = x_in;
    a.part = part;
    a.P = P;
    a.pbias = pbias;
    a.x_out = x_out;
    a.gamma = gamma;
    a.beta = beta;
    a.eps = eps;
    a.bias = bias;
    a.relu = relu ? 1 : 0;
    a.y = y;
    const size_t lds = sizeof(float) * size_t(nb) * lds_pad(d);
    return preloadable(a) ? dispatch_t<PRO_RESID_PRE, EPI_STORE, GGML_F32>(w.type, a, gemv_round_b(nb), cpl,
                                                                        gemv_grid(w, 1), lds, st)
                          : dispatch_t<PRO_RESID, EPI_STORE, GGML_F32>(w.type, a, gemv_round_b(nb), cpl, gemv_grid(w, 1),
                                                                    lds, st);
}

hipError_t step_proj(const DevMatrix &w, const float *bias, int nb, const float *x, float *y, hipStream_t st) {
    StepArgs a{};
    int cpl;
    if (!prepare(w, nb, a, &cpl) || w.K % 4) return hipErrorInvalidValue;
    a.xg = x;
    a.ldx = w.K;
    a.bias = bias;
    a.y = y;
    return dispatch_t<PRO_GLOBAL, EPI_STORE, GGML_F32>(w.type, a, gemv_round_b(nb), cpl, gemv_grid(w, 1), 0, st);
}

}  // namespace mlg
