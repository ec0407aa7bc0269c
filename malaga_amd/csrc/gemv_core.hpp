// Register-resident dequant-GEMV core (batch 1..4), shared by the plain GEMV
// kernels and the fused decoder-step kernels.
//
// Work layout (wave64): a lane owns a fixed chunk of the row (XW weights) for
// the whole kernel, so its slice of x stays in registers.  The LPR lanes of a
// row group (a power of two <= 64) stream one row with 16-byte loads; a wave
// covers 64/LPR rows per row group and handles two row groups per step.  All
// loads of a step are issued unconditionally (row and chunk indices clamped, x
// zeroed for padding chunks), and the next step's loads are issued before the
// current step is computed, so a wave keeps up to four rows in flight.  Integer
// quants are widened with v_cvt_f32_ubyteN and accumulated in f32; block
// offsets (q4_K/q5_K min, q6_K -32, q8_0 sign) are applied once per group from
// per-lane sums of x.
#pragma once
#include "device.hpp"
#include "kernels.hpp"
#include "quant.hpp"

namespace mlg {

template <int T>
struct GTraits;
template <>
struct GTraits<GGML_Q4_K> { static constexpr int XW = 64, NS = 2; };  // chunk = 64-value group g of a block
template <>
struct GTraits<GGML_Q5_K> { static constexpr int XW = 64, NS = 2; };
template <>
struct GTraits<GGML_Q6_K> { static constexpr int XW = 64, NS = 4; };  // chunk = (half, 16-lane) slice
template <>
struct GTraits<GGML_Q8_0> { static constexpr int XW = 32, NS = 1; };  // chunk = one block
template <>
struct GTraits<GGML_F16> { static constexpr int XW = 8, NS = 1; };
template <>
struct GTraits<GGML_F32> { static constexpr int XW = 4, NS = 1; };

struct WPtr {
    const uint8_t *q, *s, *d;
    int N, K, nb;  // nb: blocks per row
};

// x position of element e (0..XW-1) of chunk c
template <int T>
__device__ __forceinline__ int xpos(int c, int e) {
    if constexpr (T == GGML_Q4_K || T == GGML_Q5_K) {
        return (c >> 2) * 256 + (c & 3) * 64 + e;
    } else if constexpr (T == GGML_Q6_K) {
        return (c >> 2) * 256 + ((c >> 1) & 1) * 128 + (c & 1) * 16 + (e >> 4) * 32 + (e & 15);
    } else {
        return c * GTraits<T>::XW + e;
    }
}

template <int T>
__device__ __forceinline__ int xslot(int e) {
    if constexpr (T == GGML_Q4_K || T == GGML_Q5_K) return e >> 5;
    else if constexpr (T == GGML_Q6_K) return e >> 4;
    else return 0;
}

template <int T>
struct Raw {
    uint4 a, b, c, h, e;
    uint32_t e0, e1;
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// 16 / 8 / 2-byte loads; NT marks streaming data (read once per step, e.g. the
// 215 MB LM head) as non-temporal so that it does not evict what is reused.
template <bool NT>
__device__ __forceinline__ uint4 ld_u4(const uint8_t *p) {
    if constexpr (NT) {
        const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *reinterpret_cast<const uint4 *>(p);
    }
}
template <bool NT>
__device__ __forceinline__ uint2 ld_u2(const uint8_t *p) {
    if constexpr (NT) {
        const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p));
        return make_uint2(v.x, v.y);
    } else {
        return *reinterpret_cast<const uint2 *>(p);
    }
}
template <bool NT>
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const unsigned short *>(p));
    else return *reinterpret_cast<const unsigned short *>(p);
}

template <int T, bool NT = false>
__device__ __forceinline__ void load_chunk(const WPtr &w, int row, int c, Raw<T> &r) {
    if constexpr (T == GGML_Q4_K) {
        const uint8_t *blk = w.q + (size_t(row) * w.nb + (c >> 2)) * 144;
        const int g = c & 3;
        r.h = ld_u4<NT>(blk);
        r.a = ld_u4<NT>(blk + 16 + 32 * g);
        r.b = ld_u4<NT>(blk + 32 + 32 * g);
    } else if constexpr (T == GGML_Q5_K) {
        const uint8_t *blk = w.q + (size_t(row) * w.nb + (c >> 2)) * 176;
        const int g = c & 3;
        r.h = ld_u4<NT>(blk);
        r.c = ld_u4<NT>(blk + 16);  // qh[0..15]
        r.e = ld_u4<NT>(blk + 32);  // qh[16..31]
        r.a = ld_u4<NT>(blk + 48 + 32 * g);
        r.b = ld_u4<NT>(blk + 64 + 32 * g);
    } else if constexpr (T == GGML_Q6_K) {
        const size_t blk = size_t(row) * w.nb + (c >> 2);
        const int h2 = (c >> 1) & 1, i = c & 1;
        const uint8_t *qp = w.q + blk * 192;
        r.a = ld_u4<NT>(qp + 64 * h2 + 16 * i);
        r.b = ld_u4<NT>(qp + 64 * h2 + 32 + 16 * i);
        r.h = ld_u4<NT>(qp + 128 + 32 * h2 + 16 * i);
        const uint2 sc = ld_u2<NT>(w.s + blk * 16 + 8 * h2);
        r.e0 = sc.x;
        r.e1 = sc.y;
        r.c.x = ld_u16<NT>(w.d + blk * 2);
    } else if constexpr (T == GGML_Q8_0) {
        const uint8_t *qp = w.q + size_t(row) * w.K + 32 * c;
        r.a = ld_u4<NT>(qp);
        r.b = ld_u4<NT>(qp + 16);
        r.e0 = ld_u16<NT>(w.d + (size_t(row) * (w.K >> 5) + c) * 2);
    } else if constexpr (T == GGML_F16) {
        r.a = ld_u4<NT>(w.q + (size_t(row) * w.K + 8 * c) * 2);
    } else {
        r.a = ld_u4<NT>(w.q + (size_t(row) * w.K + 4 * c) * 4);
    }
}

template <int T, int B>
__device__ __forceinline__ void dot_chunk(int c, const Raw<T> &r, const float (&x)[B][GTraits<T>::XW],
                                          const float (&xs)[B][GTraits<T>::NS], float (&acc)[B]) {
    if constexpr (T == GGML_Q4_K || T == GGML_Q5_K) {
        const int g = c & 3;
        // scale/min of sub-blocks 2g (low nibbles) and 2g+1 (high nibbles); the 6-bit
        // table keeps sub-blocks 0..3 in bytes 0..7 and 4..7 split over bytes 8..11 + high bits
        const int sh0 = 8 * ((2 * g) & 3), sh1 = sh0 + 8;
        const bool upper = g >= 2;
        auto decode = [&](int sh, float &sc, float &mn) {
            const uint32_t B0 = r.h.y >> sh, B1 = r.h.z >> sh, B2 = r.h.w >> sh;
            const uint32_t a = upper ? ((B2 & 15u) | ((B0 >> 2) & 48u)) : (B0 & 63u);
            const uint32_t bb = upper ? (((B2 >> 4) & 15u) | ((B1 >> 2) & 48u)) : (B1 & 63u);
            sc = float(a);
            mn = float(bb);
        };
        float sc0, m0, sc1, m1;
        decode(sh0, sc0, m0);
        decode(sh1, sc1, m1);
        const float d = h2f(r.h.x), dmin = h2f(r.h.x >> 16);
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        uint32_t hb[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if constexpr (T == GGML_Q5_K) {
            hb[0] = r.c.x; hb[1] = r.c.y; hb[2] = r.c.z; hb[3] = r.c.w;
            hb[4] = r.e.x; hb[5] = r.e.y; hb[6] = r.e.z; hb[7] = r.e.w;
        }
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if constexpr (T == GGML_Q5_K) {
                lo[u] = (w[u] & 0x0F0F0F0Fu) | (((hb[u] >> (2 * g)) & 0x01010101u) << 4);
                hi[u] = ((w[u] >> 4) & 0x0F0F0F0Fu) | (((hb[u] >> (2 * g + 1)) & 0x01010101u) << 4);
            } else {
                lo[u] = w[u] & 0x0F0F0F0Fu;
                hi[u] = w[u] & 0xF0F0F0F0u;  // 16 * nibble; scaled back below
            }
        }
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            float al = 0.f, ah = 0.f;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                al = dot4u8(lo[u], &x[bi][4 * u], al);
                ah = dot4u8(hi[u], &x[bi][32 + 4 * u], ah);
            }
            if constexpr (T == GGML_Q4_K) ah *= 0.0625f;
            acc[bi] += d * (sc0 * al + sc1 * ah) - dmin * (m0 * xs[bi][0] + m1 * xs[bi][1]);
        }
    } else if constexpr (T == GGML_Q6_K) {
        const int i = c & 1;
        const float d = h2f(r.c.x);
        const float sc[4] = {float(int8_t(r.e0 >> (8 * i))), float(int8_t(r.e0 >> (8 * i + 16))),
                             float(int8_t(r.e1 >> (8 * i))), float(int8_t(r.e1 >> (8 * i + 16)))};
        const uint32_t A[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, Bq[4] = {r.b.x, r.b.y, r.b.z, r.b.w},
                       H[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
        uint32_t g0[4], g1[4], g2[4], g3[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            g0[u] = (A[u] & 0x0F0F0F0Fu) | ((H[u] << 4) & 0x30303030u);
            g1[u] = (Bq[u] & 0x0F0F0F0Fu) | ((H[u] << 2) & 0x30303030u);
            g2[u] = ((A[u] >> 4) & 0x0F0F0F0Fu) | (H[u] & 0x30303030u);
            g3[u] = ((Bq[u] >> 4) & 0x0F0F0F0Fu) | ((H[u] >> 2) & 0x30303030u);
        }
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a0 = dot4u8(g0[u], &x[bi][4 * u], a0);
                a1 = dot4u8(g1[u], &x[bi][16 + 4 * u], a1);
                a2 = dot4u8(g2[u], &x[bi][32 + 4 * u], a2);
                a3 = dot4u8(g3[u], &x[bi][48 + 4 * u], a3);
            }
            acc[bi] += d * (sc[0] * (a0 - 32.f * xs[bi][0]) + sc[1] * (a1 - 32.f * xs[bi][1]) +
                            sc[2] * (a2 - 32.f * xs[bi][2]) + sc[3] * (a3 - 32.f * xs[bi][3]));
        }
    } else if constexpr (T == GGML_Q8_0) {
        const float d = h2f(r.e0);
        const uint32_t w[8] = {r.a.x ^ 0x80808080u, r.a.y ^ 0x80808080u, r.a.z ^ 0x80808080u, r.a.w ^ 0x80808080u,
                               r.b.x ^ 0x80808080u, r.b.y ^ 0x80808080u, r.b.z ^ 0x80808080u, r.b.w ^ 0x80808080u};
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            float a = 0.f;
#pragma unroll
            for (int u = 0; u < 8; ++u) a = dot4u8(w[u], &x[bi][4 * u], a);  // (q + 128) . x
            acc[bi] += d * (a - 128.f * xs[bi][0]);
        }
    } else if constexpr (T == GGML_F16) {
        const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            float a = acc[bi];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a = fmaf(h2f(w[u]), x[bi][2 * u], a);
                a = fmaf(h2f(w[u] >> 16), x[bi][2 * u + 1], a);
            }
            acc[bi] = a;
        }
    } else {
        const float w[4] = {__uint_as_float(r.a.x), __uint_as_float(r.a.y), __uint_as_float(r.a.z),
                            __uint_as_float(r.a.w)};
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            float a = acc[bi];
#pragma unroll
            for (int u = 0; u < 4; ++u) a = fmaf(w[u], x[bi][u], a);
            acc[bi] = a;
        }
    }
}

// Lane geometry of one GEMV launch (uniform per launch).
struct GemvGeom {
    int lpr_log2;  // lanes per row group = 1 << lpr_log2 (<= 64)
    int nchunks;   // chunks per row
};

// LDS rows of x staged for the GEMV carry 4 floats of padding after every 64, so
// that the 16-byte reads of the lanes of a row group (one chunk each, 64 floats
// apart) fall in different banks.
__host__ __device__ constexpr int lds_pad(int i) { return i + ((i >> 6) << 2); }

// Loads this lane's slice of x (rows [0, nb) of a [B][ldx] array; 16-byte aligned,
// generic pointer: LDS or global) into registers; padding rows/chunks are zero.
// PAD: x is an LDS copy in the lds_pad layout.
template <int T, int B, int CPL, bool PAD = false>
__device__ __forceinline__ void gemv_load_x(const float *x, int ldx, int nb, const GemvGeom &g, int cl,
                                            float (&xr)[CPL][B][GTraits<T>::XW],
                                            float (&xs)[CPL][B][GTraits<T>::NS]) {
    constexpr int XW = GTraits<T>::XW, NS = GTraits<T>::NS;
    const int lpr = 1 << g.lpr_log2;
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
        const int c = cl + t * lpr;
        const bool valid = c < g.nchunks;
        const int cc = valid ? c : 0;
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            const bool v = valid && bi < nb;
            const float *row = x + size_t(bi < nb ? bi : 0) * ldx;
#pragma unroll
            for (int e = 0; e < XW; e += 4) {
                const int o = PAD ? lds_pad(xpos<T>(cc, e)) : xpos<T>(cc, e);
                const float4 q = *reinterpret_cast<const float4 *>(row + o);
                xr[t][bi][e] = v ? q.x : 0.f;
                xr[t][bi][e + 1] = v ? q.y : 0.f;
                xr[t][bi][e + 2] = v ? q.z : 0.f;
                xr[t][bi][e + 3] = v ? q.w : 0.f;
            }
#pragma unroll
            for (int s = 0; s < NS; ++s) xs[t][bi][s] = 0.f;
#pragma unroll
            for (int e = 0; e < XW; ++e) xs[t][bi][xslot<T>(e)] += xr[t][bi][e];
        }
    }
}

struct NoPre {
    __device__ void operator()() const {}
};

// NT: rows >= nt_from are loaded non-temporally, the rows before with cached loads.
// Streams the rows of W; calls epi(row, bi, value) on the group-leader lane of each
// row (value = dot product + bias[row], the bias fetched with the weights).  Waves
// gwave, gwave + nwaves, ... share the rows, G row groups per wave and step (two
// steps in flight).  G = 1 halves the arithmetic on a wave's critical path (small
// matrices, latency-bound); G = 2 keeps more bytes in flight (the LM head).
// Order of issue: pre() (loads the
// prologue needs, so that waiting for them does not wait for the weights: loads
// complete in order), the first step's weights, then prologue(), which fills
// xr/xs and may use workgroup barriers (every thread of the workgroup must call
// this function).
template <int T, int B, int CPL, bool NT = false, int G = 2, class PreF, class Pro, class Epi>
__device__ __forceinline__ void gemv_rows(const WPtr &w, const GemvGeom &g, float (&xr)[CPL][B][GTraits<T>::XW],
                                          float (&xs)[CPL][B][GTraits<T>::NS], int gwave, int nwaves, PreF &&pre,
                                          Pro &&prologue, Epi &epi, const float *bias = nullptr,
                                          int nt_from = 0) {
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << g.lpr_log2, rpw = 64 >> g.lpr_log2;
    const int grp = lane >> g.lpr_log2, cl = lane & (lpr - 1);
    int cidx[CPL];
#pragma unroll
    for (int t = 0; t < CPL; ++t) cidx[t] = (cl + t * lpr < g.nchunks) ? cl + t * lpr : 0;

    auto load_step = [&](int rg, Raw<T> (&r)[G][CPL], float (&bv)[G]) {
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const int row = min((rg + u * nwaves) * rpw + grp, w.N - 1);
            if (NT && (rg + u * nwaves) * rpw >= nt_from) {  // wave-uniform
#pragma unroll
                for (int t = 0; t < CPL; ++t) load_chunk<T, true>(w, row, cidx[t], r[u][t]);
            } else {
#pragma unroll
                for (int t = 0; t < CPL; ++t) load_chunk<T, false>(w, row, cidx[t], r[u][t]);
            }
            bv[u] = bias ? bias[row] : 0.f;
        }
    };
    auto compute_step = [&](int rg, const Raw<T> (&r)[G][CPL], const float (&bv)[G]) {
#pragma unroll
        for (int u = 0; u < G; ++u) {
            float acc[B];
#pragma unroll
            for (int bi = 0; bi < B; ++bi) acc[bi] = 0.f;
#pragma unroll
            for (int t = 0; t < CPL; ++t) dot_chunk<T, B>(cidx[t], r[u][t], xr[t], xs[t], acc);
#pragma unroll
            for (int bi = 0; bi < B; ++bi)
                acc[bi] = group_sum_dyn(acc[bi], g.lpr_log2);
            const int row = (rg + u * nwaves) * rpw + grp;
            if (cl == 0 && row < w.N) {
#pragma unroll
                for (int bi = 0; bi < B; ++bi) epi(row, bi, acc[bi] + bv[u]);
            }
        }
    };

    const int stride = G * nwaves;
    int rg = gwave;
    const bool any = rg * rpw < w.N;  // wave-uniform
    Raw<T> A[G][CPL], Bf[G][CPL];
    float ba[G], bb[G];
#pragma unroll
    for (int u = 0; u < G; ++u) ba[u] = bb[u] = 0.f;
    pre();
    __builtin_amdgcn_sched_barrier(0);
    if (any) load_step(rg, A, ba);
    __builtin_amdgcn_sched_barrier(0);
    prologue();
    if (!any) return;
    for (;;) {
        const int rb = rg + stride;
        const bool more_b = rb * rpw < w.N;
        if (more_b) load_step(rb, Bf, bb);
        compute_step(rg, A, ba);
        if (!more_b) break;
        rg = rb;
        const int ra = rg + stride;
        const bool more_a = ra * rpw < w.N;
        if (more_a) load_step(ra, A, ba);
        compute_step(rg, Bf, bb);
        if (!more_a) break;
        rg = ra;
    }
}

// ---- host-side geometry shared by the launchers ----

constexpr int kGemvMaxXRegs = 128;  // x values a lane keeps in registers (XW * B * CPL)

inline int gemv_xw(uint32_t t) {
    switch (t) {
    case GGML_Q4_K: case GGML_Q5_K: case GGML_Q6_K: return 64;
    case GGML_Q8_0: return 32;
    case GGML_F16: return 8;
    case GGML_F32: return 4;
    default: return 0;
    }
}

inline WPtr wptr_of(const DevMatrix &w) {
    TypeInfo ti;
    type_info(w.type, &ti);
    return WPtr{w.q, w.s, w.d, w.N, w.K, w.K / ti.block_elems};
}

// lanes per row group and chunks per lane for matrix w
inline bool gemv_geometry(const DevMatrix &w, GemvGeom *g, int *cpl) {
    const int xw = gemv_xw(w.type);
    if (!xw || w.K % xw) return false;
    const int nc = w.K / xw;
    int l2 = 0;
    while ((1 << l2) < nc && l2 < 6) ++l2;
    g->lpr_log2 = l2;
    g->nchunks = nc;
    *cpl = (nc + 63) / 64;
    return *cpl <= 4;
}

inline int gemv_round_b(int b) { return b <= 1 ? 1 : (b <= 2 ? 2 : 4); }

}  // namespace mlg
