// Row-wise and attention kernels of the decoder step and the encoder:
// LayerNorm (+ residual, + embedding/positions), q/k/v split into the f16 KV
// cache, single-query and prefill attention, argmax + greedy bookkeeping,
// log-softmax top-k for beam search, and small copy helpers.
#include <mutex>
#include <vector>

#include "dequant.hpp"
#include "kernels.hpp"

namespace mlg {

namespace {

// ---- rows: one wave per row, four rows per workgroup ----------------------------

// LayerNorm of rows (RESID: x += y first, stored back; the normalized row goes to h).
// FRAG: x in fragment order (frag_index), h row-major.
template <int NJ, bool RESID, bool FRAG = false>
__global__ __launch_bounds__(256) void k_rows_ln(float *x, const float *y, int rows, int d, const float *g,
                                                 const float *b, float eps, float *h) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform; nothing below synchronizes the workgroup
    float4 *xr = reinterpret_cast<float4 *>(x + size_t(row) * d);
    const float4 *yr = reinterpret_cast<const float4 *>(y + size_t(row) * d);
    auto form = [&](int f) {
        if constexpr (FRAG) return reinterpret_cast<const float4 *>(x)[frag_index(row, 4 * f, d)];
        float4 v = xr[f];
        if constexpr (RESID) add4(v, yr[f]);
        return v;
    };
    if constexpr (RESID) {
        wave_row_layernorm<NJ>(d, form, [&](int f, const float4 &v) { xr[f] = v; }, g, b, eps, h + size_t(row) * d);
    } else {
        wave_row_layernorm<NJ>(d, form, NoKeep{}, g, b, eps, h + size_t(row) * d);
    }
}

// Embedding rows, one wave per row: lane l owns the 16-value chunks c = l + 64 j
// (j < NC, d <= 1024 NC, d % 16 == 0), each dequantized straight into registers.
template <int T, int NC>
__device__ __forceinline__ void embed_chunks(const uint8_t *q, const uint8_t *s, const uint8_t *dp, int d,
                                             uint32_t tok, float (&w)[NC][16]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < NC; ++j)
        if (16 * (lane + 64 * j) < d) dequant16<T>(q, s, dp, d, int(tok), 16 * (lane + 64 * j), w[j]);
}

// src/model.rs:558-568: x = token_embd[id] * scale + pos[*step + base] (or, for a copied
// source token, its row of src.emb), stored to x, and h = LayerNorm(x) (decoder layer
// 0's attn_norm).  The row's values stay in registers: one pass of f64 statistics.
// SRC: a source-copy row map is given (shortlist decoding); without it no branch on it.
template <int T, int NC, bool SRC>
__global__ __launch_bounds__(256) void k_embed_pos_ln(const uint8_t *q, const uint8_t *s, const uint8_t *dp,
                                                      const uint32_t *ids, int rows, const float *pos,
                                                      const uint32_t *step, uint32_t base, float scale, int d,
                                                      uint32_t last, const float *g, const float *b, float eps,
                                                      float *x, float *h, SrcEmb src, int x_frag) {
    // row a scalar: the token id and the source-row flag are scalar loads, which do not
    // make the wave wait for the vector loads below
    const int row = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6)), lane = threadIdx.x & 63;
    if (row >= rows) return;  // wave-uniform
    const uint32_t sr = SRC ? src.row[row] : kNoRow;  // wave-uniform
    // a token the device produced: clamped to the table (an all-NaN row of logits
    // yields 0xffffffff, malaga.cu:257-258), so a bad model cannot read past it
    const uint32_t tok = min(ids[row], last), stp = *step;
    // all three read here (an empty statement that uses them): the compiler would otherwise
    // load the id only in the branch that needs it, one round trip later
    __asm__ volatile("" ::"s"(tok), "s"(sr), "s"(stp));
    // the operands that do not depend on the token first (positions; gamma and beta up to
    // d = 2048), so that their loads overlap the token's round trip instead of following
    // the embedding row one after another
    constexpr bool kGB = NC <= 2;  // gamma | beta in registers from the start
    const float *pr = pos + size_t(stp + base) * d;
    float4 pq[NC][4], gq[kGB ? NC : 1][4], bq[kGB ? NC : 1][4];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = min(lane + 64 * j, d / 16 - 1);  // lanes past d re-read the last chunk
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            pq[j][u] = ld4(pr, 4 * c + u);
            if constexpr (kGB) {
                gq[j][u] = ld4(g, 4 * c + u);
                bq[j][u] = ld4(b, 4 * c + u);
            }
        }
    }
    float w[NC][16];
    if (SRC && sr != kNoRow) {  // the previous token was a copy of source position sr
        const float *er = src.emb + (size_t(row) * src.S + sr) * d;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = lane + 64 * j;
            if (16 * c < d)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float4 v = ld4(er, 4 * c + u);
                    w[j][4 * u] = v.x;
                    w[j][4 * u + 1] = v.y;
                    w[j][4 * u + 2] = v.z;
                    w[j][4 * u + 3] = v.w;
                }
        }
    } else {
        embed_chunks<T, NC>(q, s, dp, d, tok, w);
    }
    float4 *xr = reinterpret_cast<float4 *>(x + size_t(row) * d);
    float4 v[NC][4];
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = lane + 64 * j;
        if (16 * c >= d) continue;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float4 p = pq[j][u];
            v[j][u] = make_float4(w[j][4 * u] * scale + p.x, w[j][4 * u + 1] * scale + p.y,
                                  w[j][4 * u + 2] * scale + p.z, w[j][4 * u + 3] * scale + p.w);
            if (x_frag)  // kernel argument
                reinterpret_cast<float4 *>(x)[frag_index(row, 4 * (4 * c + u), d)] = v[j][u];
            else
                xr[4 * c + u] = v[j][u];
            ln_acc(v[j][u], s1, s2);
        }
    }
    float mean, rstd;
    wave_ln_stats(s1, s2, d, eps, mean, rstd);
    float4 *hr = reinterpret_cast<float4 *>(h + size_t(row) * d);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = lane + 64 * j;
        if (16 * c >= d) continue;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if constexpr (kGB) hr[4 * c + u] = ln_apply(v[j][u], mean, rstd, gq[j][u], bq[j][u]);
            else hr[4 * c + u] = ln_apply(v[j][u], mean, rstd, ld4(g, 4 * c + u), ld4(b, 4 * c + u));
        }
    }
}

// Encoder input (src/model.rs:463-477): x = token_embd[ids[r]] * scale + pos[pidx[r]].
// scale = 0: the embedding rows alone (token_embd gathers, shortlist source rows).
template <int T, int NC>
__global__ __launch_bounds__(256) void k_embed_pos_rows(const uint8_t *q, const uint8_t *s, const uint8_t *dp,
                                                        const uint32_t *ids, const uint32_t *pidx, int rows,
                                                        const float *pos, float scale, int d, float *x) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    float w[NC][16];
    embed_chunks<T, NC>(q, s, dp, d, ids[row], w);
    const float *pr = pos ? pos + size_t(pidx[row]) * d : nullptr;
    float4 *xr = reinterpret_cast<float4 *>(x + size_t(row) * d);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = lane + 64 * j;
        if (16 * c >= d) continue;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float4 v = make_float4(w[j][4 * u], w[j][4 * u + 1], w[j][4 * u + 2], w[j][4 * u + 3]);
            if (pr) {
                const float4 p = ld4(pr, 4 * c + u);
                v = make_float4(v.x * scale + p.x, v.y * scale + p.y, v.z * scale + p.z, v.w * scale + p.w);
            }
            xr[4 * c + u] = v;
        }
    }
}

// kernels/malaga.cu:229-243 (row_dots): one wave per (row, source position).
__global__ __launch_bounds__(256) void k_source_logits(const float *h, const float *emb, const uint32_t *src_ids,
                                                       int b, int S, int d, int mask_id, int V1, float *spv,
                                                       uint32_t *spi) {
    const int p = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (p >= b * S) return;  // wave-uniform
    const int r = p / S;
    const float4 *x = reinterpret_cast<const float4 *>(h + size_t(r) * d);
    const float4 *e = reinterpret_cast<const float4 *>(emb + size_t(p) * d);
    float acc = 0.f;
    for (int t = lane; t < d / 4; t += 64) {
        const float4 a = x[t], c = e[t];
        acc += a.x * c.x + a.y * c.y + a.z * c.z + a.w * c.w;
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        spv[p] = (mask_id >= 0 && src_ids[p] == uint32_t(mask_id)) ? -INFINITY : acc;
        spi[p] = uint32_t(V1 + p % S);
    }
}

// Eight cache values from f32: f16 caches round to nearest even (one 16-byte store), f32
// caches keep the values (two 16-byte stores).
__device__ __forceinline__ void store_kv8(__half *dst, const float *p) {
    const float4 a = ld4(p, 0), z = ld4(p, 1);
    uint4 o;
    o.x = uint32_t(__half_as_ushort(__float2half(a.x))) | uint32_t(__half_as_ushort(__float2half(a.y))) << 16;
    o.y = uint32_t(__half_as_ushort(__float2half(a.z))) | uint32_t(__half_as_ushort(__float2half(a.w))) << 16;
    o.z = uint32_t(__half_as_ushort(__float2half(z.x))) | uint32_t(__half_as_ushort(__float2half(z.y))) << 16;
    o.w = uint32_t(__half_as_ushort(__float2half(z.z))) | uint32_t(__half_as_ushort(__float2half(z.w))) << 16;
    *reinterpret_cast<uint4 *>(dst) = o;
}
__device__ __forceinline__ void store_kv8(float *dst, const float *p) {
    reinterpret_cast<float4 *>(dst)[0] = ld4(p, 0);
    reinterpret_cast<float4 *>(dst)[1] = ld4(p, 1);
}

// The fused projection's rows [b][3d] (bias included) split into q (f32 [b][d]) and
// the K/V caches at slot *step ([b][H][m][hd], f16 or f32): one thread per 8 consecutive
// values of the row's d columns, two 16-byte loads per part.
template <typename KT>
__global__ __launch_bounds__(256) void k_split_qkv8(const float *qkv, int b, int H, int hd, int m,
                                                    const uint32_t *step, float *q, KT *kc, KT *vc) {
    const int d = H * hd, per_row = d / 8;
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= b * per_row) return;
    const int bi = t / per_row, c = (t - bi * per_row) * 8, hh = c / hd, e = c - hh * hd;
    const float *r = qkv + size_t(bi) * 3 * d + c;
    float4 *qd = reinterpret_cast<float4 *>(q + size_t(bi) * d + c);
    qd[0] = ld4(r, 0);
    qd[1] = ld4(r, 1);
    const size_t slot = ((size_t(bi) * H + hh) * m + *step) * hd + e;
    store_kv8(kc + slot, r + d);
    store_kv8(vc + slot, r + 2 * d);
}

// Encoder attention over the packed rows (padding positions have no row): one wave per
// (row p, head h); row p is a position of sentence i = rsent[p], whose keys and values are
// the rows soff[i] .. soff[i] + lens[i] - 1 (src/model.rs:101-109 with the padding mask).
__global__ __launch_bounds__(64) void k_attn_prefill(const float *qkv, int H, int hd, const uint32_t *soff,
                                                     const uint32_t *rsent, const uint32_t *lens, float *out) {
    extern __shared__ float sc[];
    const int id = blockIdx.x, hh = id % H, p = id / H;
    const int i = int(rsent[p]), r0 = int(soff[i]), n = int(lens[i]);
    const int d = H * hd;
    const float *qr = qkv + size_t(p) * 3 * d + hh * hd;
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < n; j += 64) {
        const float *kr = qkv + size_t(r0 + j) * 3 * d + d + hh * hd;
        float acc = 0.f;
        for (int e = 0; e < hd; e += 4) {
            const float4 a = *reinterpret_cast<const float4 *>(qr + e), b = *reinterpret_cast<const float4 *>(kr + e);
            acc = fmaf(a.x, b.x, acc);
            acc = fmaf(a.y, b.y, acc);
            acc = fmaf(a.z, b.z, acc);
            acc = fmaf(a.w, b.w, acc);
        }
        sc[j] = acc;
        mx = fmaxf(mx, acc);
    }
    mx = wave_max(mx);
    float sum = 0.f;
    for (int j = threadIdx.x; j < n; j += 64) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    __syncthreads();
    const float inv = 1.f / sum;
    for (int e = threadIdx.x; e < hd; e += 64) {
        float a = 0.f;
        for (int j = 0; j < n; ++j) a = fmaf(sc[j], qkv[size_t(r0 + j) * 3 * d + 2 * d + hh * hd + e], a);
        out[size_t(p) * d + hh * hd + e] = a * inv;
    }
}

// The stacked cross K/V projection of the packed rows, kv [Mp][L][2d] (k | v per layer), to
// the batch's per-layer [b][H][s][hd] blocks: packed row p is position prow[p] % s of
// sentence prow[p] / s.
__global__ void k_split_cross_kv(const float *kv, int Mp, const uint32_t *prow, int s, int H, int hd, int L,
                                 float *K0, size_t kv_elems) {
    const int d = H * hd;
    const size_t total = size_t(Mp) * L * d;
    for (size_t idx = blockIdx.x * size_t(blockDim.x) + threadIdx.x; idx < total; idx += size_t(gridDim.x) * blockDim.x) {
        const int c = int(idx % d);
        const size_t rest = idx / d, p = rest / L;
        const int l = int(rest % L);
        const uint32_t pr = prow[p];
        const int j = int(pr % uint32_t(s)), i = int(pr / uint32_t(s)), hh = c / hd, e = c % hd;
        const size_t dst = ((size_t(i) * H + hh) * s + j) * hd + e;
        float *K = K0 + 2 * size_t(l) * kv_elems;
        const float *src = kv + (p * L + l) * 2 * d;
        K[dst] = src[c];
        K[kv_elems + dst] = src[d + c];
    }
}

// dst row r (< n_dst) <- src row map[r] (or r when map is null)
// Every layer's cross K and V in one launch, 8 values per thread: pair p of the source
// [b][H][s][hd] (f32, as the encoder computed them) at src0 + p * src_pair -> pair p of the
// state [n][H][S][hd] (f16 for the graph step, src/graph.rs:94-97; f32 for the generic
// path) at dst0 + p * dst_pair; state row r takes source row map[r] (or r).
template <typename KT>
__global__ void k_copy_cross(const float *src0, size_t src_pair, const uint32_t *map, int n_dst, int H, int s, int hd,
                             KT *dst0, size_t dst_pair, int S, int pairs) {
    const int hv = hd / 8;
    const size_t per_row = size_t(H) * s * hv, per_pair = size_t(n_dst) * per_row, total = per_pair * pairs;
    for (size_t idx = blockIdx.x * size_t(blockDim.x) + threadIdx.x; idx < total; idx += size_t(gridDim.x) * blockDim.x) {
        const size_t p = idx / per_pair, rem0 = idx % per_pair;
        const size_t r = rem0 / per_row, rem = rem0 % per_row;
        const int ev = int(rem % hv);
        const size_t hj = rem / hv;
        const int j = int(hj % s), hh = int(hj / s);
        const size_t sr = map ? map[r] : r;
        const float *sp = src0 + p * src_pair + (sr * per_row + rem) * 8;
        KT *dp = dst0 + p * dst_pair + (((r * H + hh) * S + j) * hv + ev) * 8;
        store_kv8(dp, sp);
    }
}

__global__ __launch_bounds__(256) void k_argmax_partial(const float *logits, int V, int ldl, int chunk, int mask_id,
                                                        float *pv, uint32_t *pi) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    const int row = blockIdx.y, p = blockIdx.x, P = gridDim.x;
    const int start = p * chunk, end = min(start + chunk, V);
    const float *r = logits + size_t(row) * ldl;
    float best = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (int i = start + threadIdx.x; i < end; i += blockDim.x)
        if (i != mask_id) argmax_merge(best, bi, r[i], uint32_t(i));
    wave_argmax(best, bi);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = best;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        best = sv[0];
        bi = si[0];
        for (int k = 1; k < 4; ++k) argmax_merge(best, bi, sv[k], si[k]);
        pv[size_t(row) * P + p] = best;
        pi[size_t(row) * P + p] = bi;
    }
}

// kernels/malaga.cu:290-326 semantics (with sl.vocab_map: the shortlist mapping).
// Small batches: each row's partials are reduced by the whole workgroup (8
// independent loads per thread).
// Token of candidate i (shortlist decoding): shortlist row or source position, and
// where the next step finds its embedding (kernels/malaga.cu:309-319).
__device__ __forceinline__ uint32_t sl_token(const SlFinalize &sl, int row, uint32_t i, bool done, uint32_t pad) {
    const bool from_sl = i < uint32_t(sl.V1), from_src = !from_sl && i - uint32_t(sl.V1) < uint32_t(sl.S);
    const uint32_t tok = from_sl ? sl.vocab_map[i] : from_src ? sl.src_ids[size_t(row) * sl.S + (i - sl.V1)] : pad;
    sl.sl_row[row] = (!done && from_sl) ? i : 0u;
    sl.src_row[row] = (!done && from_src) ? i - uint32_t(sl.V1) : kNoRow;
    return tok;
}

__global__ __launch_bounds__(256) void k_greedy_finalize_wg(const float *pv, const uint32_t *pi, int P, int b,
                                                            uint8_t *finished, uint32_t *ids, uint32_t *out, int m,
                                                            uint32_t *step, uint32_t eos, uint32_t pad,
                                                            SlFinalize sl, float *outv, uint32_t *err) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t s = *step;
    for (int row = 0; row < b; ++row) {
        float best = -INFINITY;
        uint32_t bi = 0xffffffffu;
        for (int p0 = threadIdx.x; p0 < P; p0 += 256 * 8) {
            float v[8];
            uint32_t ix[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int p = p0 + u * 256;
                v[u] = p < P ? pv[size_t(row) * P + p] : -INFINITY;
                ix[u] = p < P ? pi[size_t(row) * P + p] : 0xffffffffu;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) argmax_merge(best, bi, v[u], ix[u]);
        }
        if (sl.vocab_map)  // the source-token candidates
            for (int p = threadIdx.x; p < sl.S; p += 256)
                argmax_merge(best, bi, sl.spv[size_t(row) * sl.S + p], sl.spi[size_t(row) * sl.S + p]);
        wave_argmax(best, bi);
        if (lane == 0) {
            sv[w] = best;
            si[w] = bi;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            best = sv[0];
            bi = si[0];
            for (int k = 1; k < 4; ++k) argmax_merge(best, bi, sv[k], si[k]);
            uint32_t tok = sl.vocab_map ? sl_token(sl, row, bi, finished[row] != 0, pad) : bi;
            // no finite logit in a live row (NaN from an activation past the f16 range of the
            // MFMA operands, say): reported to the host instead of decoding an arbitrary token
            if (err && !finished[row] && !(best > -INFINITY)) *err = 1u;
            if (finished[row]) tok = pad;
            if (tok == eos) finished[row] = 1;
            ids[row] = tok;
            out[size_t(row) * m + s] = tok;
            if (outv) outv[size_t(row) * m + s] = best;  // the winning logit (parity hook)
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) *step = s + 1;
}

// Larger batches: one wave per row (rows w, w + 16, ...), 8 independent loads per
// lane in flight; the step counter is advanced after every wave has read it.
__global__ __launch_bounds__(1024) void k_greedy_finalize(const float *pv, const uint32_t *pi, int P, int b,
                                                          uint8_t *finished, uint32_t *ids, uint32_t *out, int m,
                                                          uint32_t *step, uint32_t eos, uint32_t pad, SlFinalize sl,
                                                          float *outv, uint32_t *err) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint32_t s = *step;
    // two rows per pass (row0 and row0 + nw), up to 1024 partials of each requested before
    // any is merged: a wave waits for one round of loads per pass, not per 512 partials and row
    constexpr int U = 16;
    for (int row0 = w; row0 < b; row0 += 2 * nw) {  // wave-uniform
        float best[2] = {-INFINITY, -INFINITY};
        uint32_t bi[2] = {0xffffffffu, 0xffffffffu};
        for (int p0 = lane; p0 < P; p0 += 64 * U) {
            float v[2][U];
            uint32_t ix[2][U];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int row = min(row0 + r * nw, b - 1);  // a row past b reads row b - 1, unused
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int p = p0 + u * 64;
                    v[r][u] = p < P ? pv[size_t(row) * P + p] : -INFINITY;
                    ix[r][u] = p < P ? pi[size_t(row) * P + p] : 0xffffffffu;
                }
            }
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int u = 0; u < U; ++u) argmax_merge(best[r], bi[r], v[r][u], ix[r][u]);
        }
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int row = row0 + r * nw;
            if (row >= b) break;  // wave-uniform
            if (sl.vocab_map)  // the source-token candidates
                for (int p = lane; p < sl.S; p += 64)
                    argmax_merge(best[r], bi[r], sl.spv[size_t(row) * sl.S + p], sl.spi[size_t(row) * sl.S + p]);
            wave_argmax(best[r], bi[r]);
            if (lane == 0) {
                uint32_t tok = sl.vocab_map ? sl_token(sl, row, bi[r], finished[row] != 0, pad) : bi[r];
                if (err && !finished[row] && !(best[r] > -INFINITY)) *err = 1u;
                if (finished[row]) tok = pad;
                if (tok == eos) finished[row] = 1;
                ids[row] = tok;
                out[size_t(row) * m + s] = tok;
                if (outv) outv[size_t(row) * m + s] = best[r];
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) *step = s + 1;
}

// Batched decode attention, S waves per (row, head) pair (4 / S pairs per workgroup of 4
// waves): lane (split, sub) of wave q of the pair owns dimensions [8 sub, 8 sub + 8) of
// the keys SPL (S (c U + u) + q) + split, pass u < U = 8 / S of chunk c; the scores of a
// chunk feed an online softmax (running max and sum), and the wave's splits are combined
// through its LDS scratch at the end.  S = 1: no workgroup barrier; S > 1: the S partials
// (sum p_j v_j unnormalized, max, sum p_j) meet in LDS and the pair's first wave rescales
// them to their common max.
template <int HD, int S, typename KT>
__global__ __launch_bounds__(256) void k_attn_waves(const float *q, const KT *K, const KT *V, int b, int H,
                                                    int L, const uint32_t *lens, const uint32_t *step, float *out,
                                                    const uint32_t *rows, int out_split) {
    constexpr int TPK = HD / 8, SPL = 64 / TPK, U = 8 / S, SLOT = HD + 2;
    __shared__ float wsc_all[4 * 512];
    __shared__ float slots[S > 1 ? 4 * SLOT : 1];
    // w a scalar: the pair, its row and the key count stay in scalar registers
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ks = w % S, p0 = blockIdx.x * (4 / S) + w / S;
    if (S == 1 && p0 >= b * H) return;  // wave-uniform; no workgroup barrier below
    const int p = min(p0, b * H - 1);  // S > 1: a pair past the end runs on the last and is not stored
    float *wsc = wsc_all + w * 512;
    const int bi = p / H, hh = p % H, d = H * HD;
    const int sub = lane % TPK, split = lane / TPK;
    auto key = [&](int c, int u) { return SPL * (S * (c * U + u) + ks) + split; };
    // Order of issue: the first chunk's cache rows (beam's row map) and keys/values, q,
    // then the key count.  The addresses do not depend on the count (keys past it are
    // masked when used), so the chunk is not held back by that scalar read; the loads
    // complete in order.
    Kv8<KT> kr[U], vr[U];
    auto load_chunk = [&](int c) {
        size_t r[U];
        if (rows) {  // kernel argument: wave-uniform
#pragma unroll
            for (int u = 0; u < U; ++u) r[u] = rows[size_t(bi) * L + min(key(c, u), L - 1)];
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) r[u] = size_t(bi);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t o = ((r[u] * H + hh) * L + min(key(c, u), L - 1)) * HD + sub * 8;
            kr[u].load(K + o);
            vr[u].load(V + o);
        }
    };
    load_chunk(0);
    const float *qp = q + size_t(bi) * d + hh * HD + sub * 8;
    const float4 qa = *reinterpret_cast<const float4 *>(qp), qb = *reinterpret_cast<const float4 *>(qp + 4);
    __builtin_amdgcn_sched_barrier(0);
    const int n = lens ? int(lens[bi]) : int(*step) + 1;
    float m = -INFINITY, l = 0.f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int c = 0; SPL * (S * c * U + ks) < n; ++c) {  // wave-uniform; chunk 0 is in flight
        if (c) load_chunk(c);
        float sc[U];
        float cmax = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float kv[8];
            kr[u].unpack(kv);
            float sdot = kv[0] * qa.x;
            sdot = fmaf(kv[1], qa.y, sdot);
            sdot = fmaf(kv[2], qa.z, sdot);
            sdot = fmaf(kv[3], qa.w, sdot);
            sdot = fmaf(kv[4], qb.x, sdot);
            sdot = fmaf(kv[5], qb.y, sdot);
            sdot = fmaf(kv[6], qb.z, sdot);
            sdot = fmaf(kv[7], qb.w, sdot);
            sdot = group_sum<TPK>(sdot);
            sc[u] = key(c, u) < n ? sdot : -INFINITY;
            cmax = fmaxf(cmax, sc[u]);
        }
        const float mnew = fmaxf(m, wave_max(cmax));  // finite: the chunk's first key is valid
        const float rs = expf(m - mnew);
        l *= rs;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= rs;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool in = key(c, u) < n;
            const float pj = in ? expf(sc[u] - mnew) : 0.f;
            l += pj;
            float vv[8];
            vr[u].unpack(vv, in);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(pj, vv[e], acc[e]);
        }
        m = mnew;
    }
    // every lane of a split holds that split's sum: count each split once
    const float lsum = wave_sum(sub == 0 ? l : 0.f);
#pragma unroll
    for (int e = 0; e < 8; ++e) wsc[lane * 8 + e] = acc[e];
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    // output e of the pair: sum over the splits of wave q's scratch, rescaled by ew[q]
    const float *ps = S > 1 ? slots + (w - ks) * SLOT : slots;  // S > 1: the pair's partials
    float ew[S], inv;
    if constexpr (S == 1) {
        ew[0] = 1.f;
        inv = 1.f / lsum;
    } else {
        float *slot = slots + w * SLOT;
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
        __syncthreads();
        if (ks != 0 || p0 >= b * H) return;  // scalar; no barrier below
        float mx = ps[HD];  // finite: the pair's first wave has key 0
#pragma unroll
        for (int qq = 1; qq < S; ++qq) mx = fmaxf(mx, ps[qq * SLOT + HD]);
        float den = 0.f;
#pragma unroll
        for (int qq = 0; qq < S; ++qq) {
            ew[qq] = expf(ps[qq * SLOT + HD] - mx);
            den += ew[qq] * ps[qq * SLOT + HD + 1];
        }
        inv = 1.f / den;
    }
    auto value = [&](int e) {
        float o = 0.f;
        if constexpr (S == 1) {
#pragma unroll
            for (int s2 = 0; s2 < SPL; ++s2) o += wsc[(s2 * TPK + e / 8) * 8 + e % 8];
        } else {
#pragma unroll
            for (int qq = 0; qq < S; ++qq) o += ew[qq] * ps[qq * SLOT + e];
        }
        return o * inv;
    };
    if (out_split) {
        // split fragments [hi0..hi3 | lo0..lo3]: one lane per 4 values, one whole store each
        for (int e4 = lane; e4 < HD / 4; e4 += 64) {
            h4_t hv, lv;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float o = value(4 * e4 + j);
                hv[j] = _Float16(o);
                lv[j] = _Float16(o - float(hv[j]));
            }
            const uint2 hb = __builtin_bit_cast(uint2, hv), lb = __builtin_bit_cast(uint2, lv);
            reinterpret_cast<uint4 *>(out)[frag_index(bi, hh * HD + 4 * e4, d)] = make_uint4(hb.x, hb.y, lb.x, lb.y);
        }
        return;
    }
    for (int e = lane; e < HD; e += 64) out[size_t(bi) * d + hh * HD + e] = value(e);
}

// ---- log-softmax + top-k (beam search) ------------------------------------
constexpr int kTopMax = 8;
constexpr int kTopParts = 64;

// Top-8 of (value, index) pairs, best first; larger value wins, ties -> lower index.
// Always 8 entries (k <= 8 reads the first k): fixed register slots, no indexing.
struct Top8 {
    float v[kTopMax];
    uint32_t i[kTopMax];
};

__device__ __forceinline__ bool better(float av, uint32_t ai, float bv, uint32_t bi) {
    return av > bv || (av == bv && ai < bi);
}

__device__ __forceinline__ void top8_init(Top8 &t) {
#pragma unroll
    for (int j = 0; j < kTopMax; ++j) {
        t.v[j] = -INFINITY;
        t.i[j] = 0xffffffffu;
    }
}

// Without branches: c[j] = (v, i) ranks above entry j (c[j] implies c[j + 1], the list
// being sorted), so entry j becomes entry j - 1 where c[j - 1], (v, i) where c[j] alone,
// and stays otherwise; nothing changes when (v, i) does not beat the last entry.
__device__ __forceinline__ void top8_insert(Top8 &t, float v, uint32_t i) {
    bool c[kTopMax];
#pragma unroll
    for (int j = 0; j < kTopMax; ++j) c[j] = better(v, i, t.v[j], t.i[j]);
#pragma unroll
    for (int j = kTopMax - 1; j > 0; --j) {
        t.v[j] = c[j - 1] ? t.v[j - 1] : (c[j] ? v : t.v[j]);
        t.i[j] = c[j - 1] ? t.i[j - 1] : (c[j] ? i : t.i[j]);
    }
    t.v[0] = c[0] ? v : t.v[0];
    t.i[0] = c[0] ? i : t.i[0];
}

// Pass 1: per (part, row): chunk max M, sum exp(x - M), chunk top-8.
// work layout per (row, part): [M, S, v0..v7, i0..i7] (18 floats)
__global__ __launch_bounds__(256) void k_lsm_topk_partial(const float *logits, int V, int k, int mask_id,
                                                          float *work) {
    __shared__ float red[16];
    __shared__ float lv[256 * kTopMax];
    __shared__ uint32_t li[256 * kTopMax];
    const int row = blockIdx.y, p = blockIdx.x, P = gridDim.x;
    const int chunk = (V + P - 1) / P, start = p * chunk, end = min(start + chunk, V);
    const float *r = logits + size_t(row) * V;
    __shared__ float thv;
    __shared__ uint32_t thx;
    // pass 1: the thread's own best (value, index) and the chunk's max
    float bv = -INFINITY;
    uint32_t bx = 0xffffffffu;
    for (int i = start + threadIdx.x; i < end; i += blockDim.x) {
        if (i == mask_id) continue;
        const float v = r[i];
        if (better(v, uint32_t(i), bv, bx)) {
            bv = v;
            bx = uint32_t(i);
        }
    }
    lv[threadIdx.x] = bv;
    li[threadIdx.x] = bx;
    const float mx = block_max(bv, red);  // its barrier also orders lv / li
    // the chunk's 8 best are all at least as good as the 8th best of the 256 threads' bests
    // (8 distinct elements): wave 0 finds that threshold ((-inf, ~0) below 8 elements)
    if (threadIdx.x < 64) {  // wave-uniform
        const int lane = threadIdx.x;
        float hv[4];
        uint32_t hx[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            hv[q] = lv[64 * q + lane];
            hx[q] = li[64 * q + lane];
        }
        float wv = -INFINITY;
        uint32_t wx = 0xffffffffu;
#pragma unroll
        for (int rr = 0; rr < kTopMax; ++rr) {
            wv = hv[0];
            wx = hx[0];
#pragma unroll
            for (int q = 1; q < 4; ++q)
                if (better(hv[q], hx[q], wv, wx)) {
                    wv = hv[q];
                    wx = hx[q];
                }
            wave_argmax(wv, wx);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (hx[q] == wx) {
                    hv[q] = -INFINITY;
                    hx[q] = 0xffffffffu;
                }
        }
        if (lane == 0) {
            thv = wv;
            thx = wx;
        }
    }
    __syncthreads();
    const float tv = thv;
    const uint32_t tx = thx;
    // pass 2: sum exp(x - max), and a sorted top-8 of the thread's elements that reach the
    // threshold (a handful per workgroup)
    Top8 t;
    top8_init(t);
    float s = 0.f;
    for (int i = start + threadIdx.x; i < end; i += blockDim.x) {
        if (i == mask_id) continue;
        const float v = r[i];
        if (mx > -INFINITY) s += expf(v - mx);
        if (!better(tv, tx, v, uint32_t(i))) top8_insert(t, v, uint32_t(i));
    }
    s = block_sum(s, red);
    // the workgroup's best 8: the 256 sorted lists in LDS, entry e of list L at e 256 + L
    // (consecutive lanes, consecutive banks), then wave 0 takes the best head of all lists
    // 8 times: lane l keeps the heads of lists l + 64 q in registers and reads a list's next
    // entry only when its head wins.  The order is total (value, then lower index), so the
    // result is the 8 best whatever the merge order.
#pragma unroll
    for (int j = 0; j < kTopMax; ++j) {
        lv[j * 256 + threadIdx.x] = t.v[j];
        li[j * 256 + threadIdx.x] = t.i[j];
    }
    __syncthreads();
    if (threadIdx.x >= 64) return;  // wave-uniform; no barrier below
    const int lane = threadIdx.x;
    int head[4];
    float hv[4];
    uint32_t hx[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        head[q] = 0;
        hv[q] = lv[64 * q + lane];
        hx[q] = li[64 * q + lane];
    }
    float ov[kTopMax];
    uint32_t oi[kTopMax];
#pragma unroll
    for (int r = 0; r < kTopMax; ++r) {
        float bv = hv[0];
        uint32_t bx = hx[0];
#pragma unroll
        for (int q = 1; q < 4; ++q)
            if (better(hv[q], hx[q], bv, bx)) {
                bv = hv[q];
                bx = hx[q];
            }
        wave_argmax(bv, bx);
        ov[r] = bv;
        oi[r] = bx;
        // the list whose head won moves on (indices are unique; padding entries are -inf)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (hx[q] == bx && head[q] < kTopMax) {
                const int e = ++head[q];
                hv[q] = e < kTopMax ? lv[e * 256 + 64 * q + lane] : -INFINITY;
                hx[q] = e < kTopMax ? li[e * 256 + 64 * q + lane] : 0xffffffffu;
            }
    }
    if (lane == 0) {
        float *o = work + (size_t(row) * P + p) * (2 + 2 * kTopMax);
        o[0] = mx;
        o[1] = s;
#pragma unroll
        for (int j = 0; j < kTopMax; ++j) {
            o[2 + j] = ov[j];
            o[2 + kTopMax + j] = __uint_as_float(oi[j]);
        }
    }
}

// Pass 2: one wave per row, lane p holds part p (P <= 64): vals = (x - max) - ln(sum
// exp(x - max)) with the sum in f64 in a fixed lane order; top-k by k rounds of a
// wave argmax over the lanes' best remaining candidates.
__global__ __launch_bounds__(64) void k_lsm_topk_final(const float *work, int rows, int P, int k, float *vals,
                                                       uint32_t *idx) {
    const int row = blockIdx.x, lane = threadIdx.x;
    if (row >= rows) return;
    const float *o = work + (size_t(row) * P + lane) * (2 + 2 * kTopMax);
    const bool ok = lane < P;
    const float Mp = ok ? o[0] : -INFINITY, Sp = ok ? o[1] : 0.f;
    Top8 t;
    top8_init(t);
    if (ok)
#pragma unroll
        for (int j = 0; j < kTopMax; ++j) {
            t.v[j] = o[2 + j];
            t.i[j] = __float_as_uint(o[2 + kTopMax + j]);
        }
    const float M = wave_max(Mp);
    const double S = wave_sum_f64(Mp > -INFINITY ? double(Sp) * exp(double(Mp) - double(M)) : 0.0);
    const float ls = float(log(S));
    for (int j = 0; j < k; ++j) {  // uniform
        float bv = t.v[0];
        uint32_t bi = t.i[0];
        wave_argmax(bv, bi);
        if (lane == 0) {
            vals[size_t(row) * k + j] = (bv - M) - ls;
            idx[size_t(row) * k + j] = bi;
        }
        if (ok && t.i[0] == bi && t.v[0] == bv) {  // the winning lane drops its head
#pragma unroll
            for (int q = 0; q < kTopMax - 1; ++q) {
                t.v[q] = t.v[q + 1];
                t.i[q] = t.i[q + 1];
            }
            t.v[kTopMax - 1] = -INFINITY;
            t.i[kTopMax - 1] = 0xffffffffu;
        }
    }
}


__global__ void k_inc_u32(uint32_t *p) {
    if (threadIdx.x == 0) *p += 1;
}

__global__ void k_fill_u32(uint32_t *p, uint32_t v, size_t n) {
    for (size_t t = blockIdx.x * size_t(blockDim.x) + threadIdx.x; t < n; t += size_t(gridDim.x) * blockDim.x) p[t] = v;
}

int grid_1d(size_t n, int block) {
    const size_t g = (n + block - 1) / block;
    return int(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

// chunks of 16 values per lane for a row of d (<= 4096) values: 1, 2 or 4
inline int embed_nc(int d) { return d <= 1024 ? 1 : d <= 2048 ? 2 : 4; }

template <int T>
hipError_t launch_embed_pos_ln(const DevMatrix &E, const uint32_t *ids, int rows, const float *pos,
                               const uint32_t *step, uint32_t base, float scale, const float *g, const float *b,
                               float eps, float *x, float *h, hipStream_t st, const SrcEmb &src, bool x_frag) {
    const dim3 grid(unsigned((rows + 3) / 4));
    const uint32_t last = uint32_t(E.N - 1);
    const int xf = x_frag ? 1 : 0;
    switch (embed_nc(E.K)) {
    case 1:
        if (src.row)
            hipLaunchKernelGGL((k_embed_pos_ln<T, 1, true>), grid, dim3(256), 0, st, E.q, E.s, E.d, ids, rows, pos,
                               step, base, scale, E.K, last, g, b, eps, x, h, src, xf);
        else
            hipLaunchKernelGGL((k_embed_pos_ln<T, 1, false>), grid, dim3(256), 0, st, E.q, E.s, E.d, ids, rows, pos,
                               step, base, scale, E.K, last, g, b, eps, x, h, src, xf);
        break;
    case 2:
        if (src.row)
            hipLaunchKernelGGL((k_embed_pos_ln<T, 2, true>), grid, dim3(256), 0, st, E.q, E.s, E.d, ids, rows, pos,
                               step, base, scale, E.K, last, g, b, eps, x, h, src, xf);
        else
            hipLaunchKernelGGL((k_embed_pos_ln<T, 2, false>), grid, dim3(256), 0, st, E.q, E.s, E.d, ids, rows, pos,
                               step, base, scale, E.K, last, g, b, eps, x, h, src, xf);
        break;
    default:
        if (src.row)
            hipLaunchKernelGGL((k_embed_pos_ln<T, 4, true>), grid, dim3(256), 0, st, E.q, E.s, E.d, ids, rows, pos,
                               step, base, scale, E.K, last, g, b, eps, x, h, src, xf);
        else
            hipLaunchKernelGGL((k_embed_pos_ln<T, 4, false>), grid, dim3(256), 0, st, E.q, E.s, E.d, ids, rows, pos,
                               step, base, scale, E.K, last, g, b, eps, x, h, src, xf);
    }
    return hipGetLastError();
}

template <int T>
hipError_t launch_embed_pos_rows(const DevMatrix &E, const uint32_t *ids, const uint32_t *pidx, int rows,
                                 const float *pos, float scale, float *x, hipStream_t st) {
    const dim3 grid(unsigned((rows + 3) / 4));
    switch (embed_nc(E.K)) {
    case 1:
        hipLaunchKernelGGL((k_embed_pos_rows<T, 1>), grid, dim3(256), 0, st, E.q, E.s, E.d, ids, pidx, rows, pos,
                           scale, E.K, x);
        break;
    case 2:
        hipLaunchKernelGGL((k_embed_pos_rows<T, 2>), grid, dim3(256), 0, st, E.q, E.s, E.d, ids, pidx, rows, pos,
                           scale, E.K, x);
        break;
    default:
        hipLaunchKernelGGL((k_embed_pos_rows<T, 4>), grid, dim3(256), 0, st, E.q, E.s, E.d, ids, pidx, rows, pos,
                           scale, E.K, x);
    }
    return hipGetLastError();
}

template <bool RESID, bool FRAG = false>
hipError_t launch_rows_ln(float *x, const float *y, int rows, int d, const float *g, const float *b, float eps,
                          float *h, hipStream_t st) {
    if (d % 4 || d > kWaveLnMaxD || (FRAG && d % 16)) return hipErrorInvalidValue;
    if (rows <= 0) return hipSuccess;
    const dim3 grid(unsigned((rows + 3) / 4));
    const int nj = (d + 255) / 256;
    if (nj <= 1) hipLaunchKernelGGL((k_rows_ln<1, RESID, FRAG>), grid, dim3(256), 0, st, x, y, rows, d, g, b, eps, h);
    else if (nj <= 2) hipLaunchKernelGGL((k_rows_ln<2, RESID, FRAG>), grid, dim3(256), 0, st, x, y, rows, d, g, b, eps, h);
    else if (nj <= 4) hipLaunchKernelGGL((k_rows_ln<4, RESID, FRAG>), grid, dim3(256), 0, st, x, y, rows, d, g, b, eps, h);
    else if (nj <= 8) hipLaunchKernelGGL((k_rows_ln<8, RESID, FRAG>), grid, dim3(256), 0, st, x, y, rows, d, g, b, eps, h);
    else hipLaunchKernelGGL((k_rows_ln<16, RESID, FRAG>), grid, dim3(256), 0, st, x, y, rows, d, g, b, eps, h);
    return hipGetLastError();
}

}  // namespace

namespace {
// Streaming read (measurement): each thread keeps kStreamDepth 16-byte loads in flight
// over a grid-stride walk of the buffer; the words are folded into one value that is
// stored only if it matches a constant, so the loads cannot be removed.
constexpr int kStreamDepth = 8;
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
template <int MODE>
__global__ __launch_bounds__(256) void k_stream_read(const uint4 *__restrict__ p, size_t n16, uint32_t *out) {
    __shared__ uint4 stage[MODE == 2 ? 256 * kStreamDepth : 1];
    const size_t stride = size_t(gridDim.x) * 256 * kStreamDepth;
    uint32_t acc = 0;
    for (size_t base = size_t(blockIdx.x) * 256 * kStreamDepth; base < n16; base += stride) {
        if constexpr (MODE == 2) {
#pragma unroll
            for (int u = 0; u < kStreamDepth; ++u) {
                const size_t i = base + size_t(u) * 256 + threadIdx.x;
                if (i < n16)  // the LDS address is the wave's base: lane l writes 16 bytes at base + 16 l
                    __builtin_amdgcn_global_load_lds(
                        static_cast<const void *>(p + i),
                        (__attribute__((address_space(3))) void *)(stage + u * 256 + (threadIdx.x & ~63u)), 16, 0, 0);
            }
            __builtin_amdgcn_s_waitcnt(0);
            acc ^= stage[(threadIdx.x * 7) % (256 * kStreamDepth)].x;
        } else {
            uint4 v[kStreamDepth];
#pragma unroll
            for (int u = 0; u < kStreamDepth; ++u) {
                const size_t i = base + size_t(u) * 256 + threadIdx.x;
                v[u] = make_uint4(0u, 0u, 0u, 0u);
                if (i < n16) {
                    if constexpr (MODE == 1) {
                        const u32x4_v t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_v *>(p + i));
                        v[u] = make_uint4(t.x, t.y, t.z, t.w);
                    } else {
                        v[u] = p[i];
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < kStreamDepth; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        }
    }
    if (acc == 0x9e3779b9u) out[0] = acc;
}
}  // namespace

hipError_t stream_read(const void *p, size_t bytes, int mode, int grid, uint32_t *out, hipStream_t st) {
    if (!p || !out || bytes % 16 || reinterpret_cast<uintptr_t>(p) % 16 || grid < 1 || grid > 65536 || mode < 0 ||
        mode > 2)
        return hipErrorInvalidValue;
    const uint4 *q = static_cast<const uint4 *>(p);
    const size_t n16 = bytes / 16;
    if (mode == 0) hipLaunchKernelGGL(k_stream_read<0>, dim3(grid), dim3(256), 0, st, q, n16, out);
    else if (mode == 1) hipLaunchKernelGGL(k_stream_read<1>, dim3(grid), dim3(256), 0, st, q, n16, out);
    else hipLaunchKernelGGL(k_stream_read<2>, dim3(grid), dim3(256), 0, st, q, n16, out);
    return hipGetLastError();
}

hipError_t layernorm_frag(const float *x, int rows, int d, const float *g, const float *b, float eps, float *out,
                          hipStream_t st) {
    return launch_rows_ln<false, true>(const_cast<float *>(x), nullptr, rows, d, g, b, eps, out, st);
}

hipError_t layernorm(const float *x, int rows, int d, const float *g, const float *b, float eps, float *out,
                     hipStream_t st) {
    return launch_rows_ln<false>(const_cast<float *>(x), nullptr, rows, d, g, b, eps, out, st);
}

hipError_t residual_ln(float *x, const float *y, int rows, int d, const float *g, const float *b, float eps, float *h,
                       hipStream_t st) {
    return launch_rows_ln<true>(x, y, rows, d, g, b, eps, h, st);
}

hipError_t embed_pos_ln(const DevMatrix &E, const uint32_t *ids, int rows, const float *pos, const uint32_t *step,
                        uint32_t base, float scale, const float *g, const float *b, float eps, float *x, float *h,
                        hipStream_t st, const SrcEmb &src, bool x_frag) {
    if (E.K > kWaveLnMaxD || E.K % 16 || (src.row && (!src.emb || src.S < 1))) return hipErrorInvalidValue;
    if (rows <= 0) return hipSuccess;
    MLG_DISPATCH_TYPE(E.type, launch_embed_pos_ln, E, ids, rows, pos, step, base, scale, g, b, eps, x, h, st, src,
                      x_frag)
}

hipError_t embed_rows(const DevMatrix &E, const uint32_t *ids, int rows, float *out, hipStream_t st) {
    if (E.K % 16 || E.K > kWaveLnMaxD) return hipErrorInvalidValue;
    if (rows <= 0) return hipSuccess;
    MLG_DISPATCH_TYPE(E.type, launch_embed_pos_rows, E, ids, nullptr, rows, nullptr, 0.f, out, st)
}

hipError_t source_logits(const float *h, const float *emb, const uint32_t *src_ids, int b, int S, int d, int mask_id,
                         int V1, float *spv, uint32_t *spi, hipStream_t st) {
    if (d % 4 || S < 1 || b < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_source_logits, dim3(unsigned((b * S + 3) / 4)), dim3(256), 0, st, h, emb, src_ids, b, S, d,
                       mask_id, V1, spv, spi);
    return hipGetLastError();
}

hipError_t embed_pos_rows(const DevMatrix &E, const uint32_t *ids, const uint32_t *pidx, int rows, const float *pos,
                          float scale, float *x, hipStream_t st) {
    if (E.K % 16 || E.K > kWaveLnMaxD || !pos || !pidx) return hipErrorInvalidValue;
    if (rows <= 0) return hipSuccess;
    MLG_DISPATCH_TYPE(E.type, launch_embed_pos_rows, E, ids, pidx, rows, pos, scale, x, st)
}

namespace {
template <typename KT>
hipError_t qkv_split_t(const float *qkv, int b, int H, int hd, int m, const uint32_t *step, float *q, KT *kc, KT *vc,
                       hipStream_t st) {
    if (hd % 8 || b <= 0) return b <= 0 ? hipSuccess : hipErrorInvalidValue;
    const int n = b * H * hd / 8;
    hipLaunchKernelGGL(k_split_qkv8<KT>, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, qkv, b, H, hd, m, step, q,
                       kc, vc);
    return hipGetLastError();
}
}  // namespace

hipError_t qkv_split(const float *qkv, int b, int H, int hd, int m, const uint32_t *step, float *q, __half *kc,
                     __half *vc, hipStream_t st) {
    return qkv_split_t(qkv, b, H, hd, m, step, q, kc, vc, st);
}

hipError_t qkv_split(const float *qkv, int b, int H, int hd, int m, const uint32_t *step, float *q, float *kc,
                     float *vc, hipStream_t st) {
    return qkv_split_t(qkv, b, H, hd, m, step, q, kc, vc, st);
}

constexpr int kAttnSplit = 4;  // waves per (row, head) pair in k_attn_waves

bool attn_head_size_supported(int hd) {
    return hd == 8 || hd == 16 || hd == 32 || hd == 64 || hd == 128 || hd == 256;
}

namespace {
template <typename KT>
hipError_t attn_decode_t(const float *q, const KT *K, const KT *V, int b, int H, int hd, int L, const uint32_t *lens,
                         const uint32_t *step, float *out, hipStream_t st, const uint32_t *rows, bool out_split) {
    if (b * H <= 0) return hipSuccess;
    if (out_split && ((H * hd) % 16 || reinterpret_cast<uintptr_t>(out) % 16)) return hipErrorInvalidValue;
    constexpr int ppw = 4 / kAttnSplit;  // pairs per workgroup of 4 waves
    const dim3 wgrid(unsigned((b * H + ppw - 1) / ppw));
    switch (hd) {
#define MLG_ATTN_WAVES(HD)                                                                                          \
    case HD:                                                                                                        \
        hipLaunchKernelGGL((k_attn_waves<HD, kAttnSplit, KT>), wgrid, dim3(256), 0, st, q, K, V, b, H, L, lens,     \
                           step, out, rows, out_split ? 1 : 0);                                                     \
        return hipGetLastError();
        MLG_ATTN_WAVES(8)
        MLG_ATTN_WAVES(16)
        MLG_ATTN_WAVES(32)
        MLG_ATTN_WAVES(64)
        MLG_ATTN_WAVES(128)
        MLG_ATTN_WAVES(256)
#undef MLG_ATTN_WAVES
    default: return hipErrorInvalidValue;  // attn_head_size_supported is checked at model load
    }
}
}  // namespace

hipError_t attn_decode(const float *q, const __half *K, const __half *V, int b, int H, int hd, int L,
                       const uint32_t *lens, const uint32_t *step, float *out, hipStream_t st, const uint32_t *rows,
                       bool out_split) {
    return attn_decode_t(q, K, V, b, H, hd, L, lens, step, out, st, rows, out_split);
}

hipError_t attn_decode(const float *q, const float *K, const float *V, int b, int H, int hd, int L,
                       const uint32_t *lens, const uint32_t *step, float *out, hipStream_t st, const uint32_t *rows,
                       bool out_split) {
    return attn_decode_t(q, K, V, b, H, hd, L, lens, step, out, st, rows, out_split);
}

hipError_t attn_prefill(const float *qkv, int Mp, int H, int hd, const uint32_t *soff, const uint32_t *rsent,
                        const uint32_t *lens, int max_len, float *out, hipStream_t st) {
    if (hd % 4) return hipErrorInvalidValue;
    if (Mp <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_attn_prefill, dim3(unsigned(Mp) * unsigned(H)), dim3(64), sizeof(float) * max_len, st, qkv, H,
                       hd, soff, rsent, lens, out);
    return hipGetLastError();
}

hipError_t split_cross_kv(const float *kv, int Mp, const uint32_t *prow, int s, int H, int hd, int L, float *K0,
                          size_t kv_elems, hipStream_t st) {
    const size_t n = size_t(Mp) * H * hd * L;
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_split_cross_kv, dim3(grid_1d(n, 256)), dim3(256), 0, st, kv, Mp, prow, s, H, hd, L, K0,
                       kv_elems);
    return hipGetLastError();
}

namespace {
template <typename KT>
hipError_t copy_cross_t(const float *src0, size_t src_pair, const uint32_t *map, int n_dst, int H, int s, int hd,
                        KT *dst0, size_t dst_pair, int S, int pairs, hipStream_t st) {
    if (hd % 8 || src_pair % 8 || dst_pair % 8 || reinterpret_cast<uintptr_t>(src0) % 16 ||
        reinterpret_cast<uintptr_t>(dst0) % 16 || s > S)
        return hipErrorInvalidValue;
    const size_t total = size_t(pairs) * n_dst * H * s * (hd / 8);
    if (!total) return hipSuccess;
    hipLaunchKernelGGL(k_copy_cross<KT>, dim3(grid_1d(total, 256)), dim3(256), 0, st, src0, src_pair, map, n_dst, H, s,
                       hd, dst0, dst_pair, S, pairs);
    return hipGetLastError();
}
}  // namespace

hipError_t copy_cross(const float *src0, size_t src_pair, const uint32_t *map, int n_dst, int H, int s, int hd,
                      __half *dst0, size_t dst_pair, int S, int pairs, hipStream_t st) {
    return copy_cross_t(src0, src_pair, map, n_dst, H, s, hd, dst0, dst_pair, S, pairs, st);
}

hipError_t copy_cross(const float *src0, size_t src_pair, const uint32_t *map, int n_dst, int H, int s, int hd,
                      float *dst0, size_t dst_pair, int S, int pairs, hipStream_t st) {
    return copy_cross_t(src0, src_pair, map, n_dst, H, s, hd, dst0, dst_pair, S, pairs, st);
}

hipError_t argmax_partial(const float *logits, int b, int V, int ldl, int mask_id, float *pv, uint32_t *pi, int parts,
                          hipStream_t st) {
    const int chunk = (V + parts - 1) / parts;
    hipLaunchKernelGGL(k_argmax_partial, dim3(parts, b), dim3(256), 0, st, logits, V, ldl, chunk, mask_id, pv, pi);
    return hipGetLastError();
}

hipError_t greedy_finalize(const float *pv, const uint32_t *pi, int parts, int b, uint8_t *finished, uint32_t *ids,
                           uint32_t *out, int m, uint32_t *step, uint32_t eos, uint32_t pad, hipStream_t st,
                           const SlFinalize &sl, float *outv, uint32_t *err) {
    if (sl.vocab_map && (!sl.spv || !sl.spi || !sl.src_ids || !sl.sl_row || !sl.src_row || sl.S < 1))
        return hipErrorInvalidValue;
    if (b <= 4)
        hipLaunchKernelGGL(k_greedy_finalize_wg, dim3(1), dim3(256), 0, st, pv, pi, parts, b, finished, ids, out, m,
                           step, eos, pad, sl, outv, err);
    else
        hipLaunchKernelGGL(k_greedy_finalize, dim3(1), dim3(1024), 0, st, pv, pi, parts, b, finished, ids, out, m,
                           step, eos, pad, sl, outv, err);
    return hipGetLastError();
}

size_t logsoftmax_topk_scratch(int rows, int k) {
    (void)k;
    return size_t(rows) * kTopParts * (2 + 2 * kTopMax) * sizeof(float);
}

hipError_t logsoftmax_topk(const float *logits, int rows, int V, int k, int mask_id, float *work, float *vals,
                           uint32_t *idx, hipStream_t st) {
    if (k < 1 || k > kTopMax) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_lsm_topk_partial, dim3(kTopParts, rows), dim3(256), 0, st, logits, V, k, mask_id, work);
    hipLaunchKernelGGL(k_lsm_topk_final, dim3(rows), dim3(64), 0, st, work, rows, kTopParts, k, vals, idx);
    return hipGetLastError();
}


// ---- log-softmax + top-k without allocation ----------------------------------------
// The work area of logsoftmax_topk for up to kStaticTopkRows rows (1.125 MiB), a static
// device array: every GPU the library runs on holds its own copy until the process
// ends.  In host code `scratch` names a host-side stand-in, never a device address:
// only the pointer hipGetSymbolAddress returns (per device) reaches a kernel.  Nothing
// needs clearing between calls (pass 1 writes every (row, part) entry pass 2 reads);
// calls that overlap on one GPU share the array and race.
static __device__ __align__(256) float scratch[size_t(kStaticTopkRows) * kTopParts * (2 + 2 * kTopMax)];

namespace {
std::mutex g_scratch_mu;
std::vector<float *> g_scratch_dev;  // device address of `scratch`, per device

hipError_t static_scratch(float **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (size_t(dev) >= g_scratch_dev.size()) g_scratch_dev.resize(size_t(dev) + 1, nullptr);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_dev[dev] = static_cast<float *>(p);
    }
    *out = g_scratch_dev[dev];
    return hipSuccess;
}
}  // namespace

hipError_t logsoftmax_topk_static(const float *logits, int rows, int V, int k, int mask_id, float *vals, uint32_t *idx,
                                  hipStream_t st) {
    if (rows < 1 || rows > kStaticTopkRows || logsoftmax_topk_scratch(rows, k) > sizeof(scratch))
        return hipErrorInvalidValue;
    // the array's address is the current device's: a stream of another device is refused
    // (the null stream belongs to the current device)
    if (st) {
        int cur = 0;
        hipDevice_t sdev = 0;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess) e = hipStreamGetDevice(st, &sdev);
        if (e != hipSuccess) return e;
        if (int(sdev) != cur) return hipErrorInvalidValue;
    }
    float *work = nullptr;
    const hipError_t e = static_scratch(&work);
    if (e != hipSuccess) return e;
    return logsoftmax_topk(logits, rows, V, k, mask_id, work, vals, idx, st);
}

hipError_t inc_u32(uint32_t *p, hipStream_t st) {
    hipLaunchKernelGGL(k_inc_u32, dim3(1), dim3(64), 0, st, p);
    return hipGetLastError();
}

hipError_t fill_u32(uint32_t *p, uint32_t v, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_1d(n, 256)), dim3(256), 0, st, p, v, n);
    return hipGetLastError();
}

}  // namespace mlg
