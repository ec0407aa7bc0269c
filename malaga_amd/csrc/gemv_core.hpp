// Register-resident dequant-GEMV core (batch 1..4), shared by the plain GEMV
// kernels and the fused decoder-step kernels.
//
// Work layout (wave64): a lane owns a fixed chunk of the row (XW weights) for
// the whole kernel, so its slice of x stays in registers.  The LPR lanes of a
// row group (a power of two <= 64) stream one row with 16-byte loads; a wave
// covers 64/LPR rows per row group and handles two row groups per step.  All
// loads of a step are issued unconditionally (row and chunk indices clamped, x
// zeroed for padding chunks), and the next step's loads are issued before the
// current step is computed, so a wave keeps up to four rows in flight.
//
// Arithmetic.  In the large streaming GEMVs (the LM head) with integer formats
// (q4_K, q5_K, q6_K, q8_0), x is held as three balanced signed 8-bit limbs per
// value, x = s (c0 + 2^8 c1 + 2^16 c2), with one power-of-two scale s per group of
// values (256 for the k-quants, 32 for q8_0) chosen so that |x / s| < 2^22.  The products of the integer quants with
// the limbs are exact in int32 (v_dot4_i32_i8, four weights per instruction and
// limb); the three limb sums of a sub-block are combined in f32 and scaled by
// the block's scales.  This is the f32 dequantized product up to the 2^-23
// relative rounding of x to its limbs, at about half the instructions per
// weight of widening each quant to f32.  The small latency-bound GEMVs (and
// F16/F32 weights) widen the quants with v_cvt_f32_ubyteN and use f32 FMAs on x:
// there the conversion of x to limbs and its barrier would sit on the critical
// path, which costs more than the arithmetic saves (measured on the fused step).
#pragma once
#include <type_traits>

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
    const uint8_t *t = nullptr;  // the tile-major copy (DevMatrix::tm), or null
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

// ---- x of one chunk (and batch rows 0..B-1) as the dot products read it ----

template <int T>
constexpr bool kLimbX = T == GGML_Q4_K || T == GGML_Q5_K || T == GGML_Q6_K || T == GGML_Q8_0;

// f32 x: XW values and NS partial sums (F16/F32 weights; the attention-head projection)
template <int T, int B>
struct XF {
    float x[B][GTraits<T>::XW];
    float s[B][GTraits<T>::NS];
};

// limb x (integer formats): c[b][l][j] packs limb l of values 4j..4j+3 of the chunk
template <int T, int B>
struct XQ {
    static constexpr int NW = GTraits<T>::XW / 4;
    int c[B][3][NW];
    float sc[B];         // scale s of the chunk's group
    float ms[B][2];      // q4_K/q5_K: sum of x over each 32-value sub-block (min term)
    int init[B][4][3];   // q6_K: -32 * (sum of limb l over 16-value group g)
};

// LIMB: the large streaming GEMVs (LM head) take limb x; small latency-bound ones
// keep f32 x, whose staging adds nothing to the critical path
template <int T, int B, bool LIMB>
using XRep = std::conditional_t<LIMB && kLimbX<T>, XQ<T, B>, XF<T, B>>;

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

// LM (q6_K only): w.q is the lane-major copy of the quant plane (layout_lane_major), so
// the 16 lanes of a row group read 256 contiguous bytes per load; with the block-major
// plane each load leaves gaps in the cache lines it touches, which made non-temporal
// loads ~25% slower (measured on the 600M head).
template <int T, bool NT = false, bool LM = false>
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
        if constexpr (LM) {
            const size_t o = (size_t(row) * w.nb * 4 + c) * 16, P = size_t(w.N) * w.nb * 64;
            r.a = ld_u4<NT>(w.q + o);
            r.b = ld_u4<NT>(w.q + P + o);
            r.h = ld_u4<NT>(w.q + 2 * P + o);
        } else {
            const uint8_t *qp = w.q + blk * 192;
            r.a = ld_u4<NT>(qp + 64 * h2 + 16 * i);
            r.b = ld_u4<NT>(qp + 64 * h2 + 32 + 16 * i);
            r.h = ld_u4<NT>(qp + 128 + 32 * h2 + 16 * i);
        }
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
__device__ __forceinline__ void dot_chunk(int c, const Raw<T> &r, const XF<T, B> &X, float (&acc)[B]) {
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
                al = dot4u8(lo[u], &X.x[bi][4 * u], al);
                ah = dot4u8(hi[u], &X.x[bi][32 + 4 * u], ah);
            }
            if constexpr (T == GGML_Q4_K) ah *= 0.0625f;
            acc[bi] += d * (sc0 * al + sc1 * ah) - dmin * (m0 * X.s[bi][0] + m1 * X.s[bi][1]);
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
                a0 = dot4u8(g0[u], &X.x[bi][4 * u], a0);
                a1 = dot4u8(g1[u], &X.x[bi][16 + 4 * u], a1);
                a2 = dot4u8(g2[u], &X.x[bi][32 + 4 * u], a2);
                a3 = dot4u8(g3[u], &X.x[bi][48 + 4 * u], a3);
            }
            acc[bi] += d * (sc[0] * (a0 - 32.f * X.s[bi][0]) + sc[1] * (a1 - 32.f * X.s[bi][1]) +
                            sc[2] * (a2 - 32.f * X.s[bi][2]) + sc[3] * (a3 - 32.f * X.s[bi][3]));
        }
    } else if constexpr (T == GGML_Q8_0) {
        const float d = h2f(r.e0);
        const uint32_t w[8] = {r.a.x ^ 0x80808080u, r.a.y ^ 0x80808080u, r.a.z ^ 0x80808080u, r.a.w ^ 0x80808080u,
                               r.b.x ^ 0x80808080u, r.b.y ^ 0x80808080u, r.b.z ^ 0x80808080u, r.b.w ^ 0x80808080u};
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            float a = 0.f;
#pragma unroll
            for (int u = 0; u < 8; ++u) a = dot4u8(w[u], &X.x[bi][4 * u], a);  // (q + 128) . x
            acc[bi] += d * (a - 128.f * X.s[bi][0]);
        }
    } else if constexpr (T == GGML_F16) {
        const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            float a = acc[bi];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a = fmaf(h2f(w[u]), X.x[bi][2 * u], a);
                a = fmaf(h2f(w[u] >> 16), X.x[bi][2 * u + 1], a);
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
            for (int u = 0; u < 4; ++u) a = fmaf(w[u], X.x[bi][u], a);
            acc[bi] = a;
        }
    }
}

__device__ __forceinline__ int sdot4(uint32_t a, int b, int c) { return __builtin_amdgcn_sdot4(int(a), b, c, false); }

// s0 + 2^8 s1 + 2^16 s2 of three limb sums, in f32
__device__ __forceinline__ float limb_sum(int s0, int s1, int s2) { return float(s0 + (s1 << 8)) + 65536.f * float(s2); }

template <int T, int B>
__device__ __forceinline__ void dot_chunk(int c, const Raw<T> &r, const XQ<T, B> &X, float (&acc)[B]) {
    if constexpr (T == GGML_Q4_K || T == GGML_Q5_K) {
        const int g = c & 3;
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
        const uint32_t hb[8] = {r.c.x, r.c.y, r.c.z, r.c.w, r.e.x, r.e.y, r.e.z, r.e.w};  // q5_K fifth bits
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if constexpr (T == GGML_Q5_K) {
                lo[u] = (w[u] & 0x0F0F0F0Fu) | (((hb[u] >> (2 * g)) & 0x01010101u) << 4);
                hi[u] = ((w[u] >> 4) & 0x0F0F0F0Fu) | (((hb[u] >> (2 * g + 1)) & 0x01010101u) << 4);
            } else {
                lo[u] = w[u] & 0x0F0F0F0Fu;
                hi[u] = (w[u] >> 4) & 0x0F0F0F0Fu;
            }
        }
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                a0 = sdot4(lo[u], X.c[bi][0][u], a0);
                a1 = sdot4(lo[u], X.c[bi][1][u], a1);
                a2 = sdot4(lo[u], X.c[bi][2][u], a2);
                b0 = sdot4(hi[u], X.c[bi][0][8 + u], b0);
                b1 = sdot4(hi[u], X.c[bi][1][8 + u], b1);
                b2 = sdot4(hi[u], X.c[bi][2][8 + u], b2);
            }
            acc[bi] += d * X.sc[bi] * (sc0 * limb_sum(a0, a1, a2) + sc1 * limb_sum(b0, b1, b2)) -
                       dmin * (m0 * X.ms[bi][0] + m1 * X.ms[bi][1]);
        }
    } else if constexpr (T == GGML_Q6_K) {
        const int i = c & 1;
        const float d = h2f(r.c.x);
        const int sc[4] = {int(int8_t(r.e0 >> (8 * i))), int(int8_t(r.e0 >> (8 * i + 16))),
                           int(int8_t(r.e1 >> (8 * i))), int(int8_t(r.e1 >> (8 * i + 16)))};
        const uint32_t A[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, Bq[4] = {r.b.x, r.b.y, r.b.z, r.b.w},
                       H[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
        uint32_t q6[4][4];  // 6-bit quants (0..63) of the four 16-value groups
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            q6[0][u] = (A[u] & 0x0F0F0F0Fu) | ((H[u] << 4) & 0x30303030u);
            q6[1][u] = (Bq[u] & 0x0F0F0F0Fu) | ((H[u] << 2) & 0x30303030u);
            q6[2][u] = ((A[u] >> 4) & 0x0F0F0F0Fu) | (H[u] & 0x30303030u);
            q6[3][u] = ((Bq[u] >> 4) & 0x0F0F0F0Fu) | ((H[u] >> 2) & 0x30303030u);
        }
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            // per limb, sum over groups of scale * (sum (q6 - 32) * limb) in int32:
            // |group sum| <= 16 * 32 * 128 = 2^16, |scale| <= 128, four groups < 2^25
            int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // sum (q6 - 32) * limb: the -32 term is the accumulator's start value
                int a0 = X.init[bi][q][0], a1 = X.init[bi][q][1], a2 = X.init[bi][q][2];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    a0 = sdot4(q6[q][u], X.c[bi][0][4 * q + u], a0);
                    a1 = sdot4(q6[q][u], X.c[bi][1][4 * q + u], a1);
                    a2 = sdot4(q6[q][u], X.c[bi][2][4 * q + u], a2);
                }
                t0 += __mul24(a0, sc[q]);
                t1 += __mul24(a1, sc[q]);
                t2 += __mul24(a2, sc[q]);
            }
            acc[bi] += d * X.sc[bi] * fmaf(65536.f, float(t2), fmaf(256.f, float(t1), float(t0)));
        }
    } else {  // q8_0: signed 8-bit quants
        const float d = h2f(r.e0);
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                a0 = sdot4(w[u], X.c[bi][0][u], a0);
                a1 = sdot4(w[u], X.c[bi][1][u], a1);
                a2 = sdot4(w[u], X.c[bi][2][u], a2);
            }
            acc[bi] += d * X.sc[bi] * limb_sum(a0, a1, a2);
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
                                            XF<T, B> (&xr)[CPL]) {
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
                xr[t].x[bi][e] = v ? q.x : 0.f;
                xr[t].x[bi][e + 1] = v ? q.y : 0.f;
                xr[t].x[bi][e + 2] = v ? q.z : 0.f;
                xr[t].x[bi][e + 3] = v ? q.w : 0.f;
            }
#pragma unroll
            for (int s = 0; s < NS; ++s) xr[t].s[bi][s] = 0.f;
#pragma unroll
            for (int e = 0; e < XW; ++e) xr[t].s[bi][xslot<T>(e)] += xr[t].x[bi][e];
        }
    }
}

// ---- limb x in LDS ----
//
// Row b of a staged x occupies xq_row_words(K) words: limb l of value word j
// (values 4j..4j+3) at l * xq_lw(K) + lq_pad(j), then one f32 scale per group of
// kScaleWords words.  4 words of padding after every 16 spread the 16-byte reads
// of a row group's lanes (16 words apart) over the banks.

template <int T>
constexpr int kScaleWords = T == GGML_Q8_0 ? 8 : 64;  // value words per scale: q8_0 block / k-quant super-block

__host__ __device__ constexpr int lq_pad(int j) { return j + ((j >> 4) << 2); }
__host__ __device__ constexpr int xq_lw(int K) { return lq_pad(K / 4 - 1) + 1; }
template <int T>
__host__ __device__ constexpr int xq_row_words(int K) {
    return (3 * xq_lw(K) + K / (4 * kScaleWords<T>) + 3) & ~3;
}
template <int T>
__host__ __device__ constexpr int xq_lds_bytes(int K, int nb) {
    return 4 * nb * xq_row_words<T>(K);
}

// Limbs of four values of one scale group.  Every lane of the wave must call this
// (group maximum over SW lanes); a group of SW lanes shares the scale.
template <int SW>
__device__ __forceinline__ void limbs4(const float4 v, uint32_t &w0, uint32_t &w1, uint32_t &w2, float &scale) {
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    m = group_reduce(m, SW == 64 ? 6 : 3, OpMax{});
    int E;
    (void)frexpf(m, &E);  // m < 2^E
    const int e = m > 0.f ? 22 - E : 0;
    const float vv[4] = {v.x, v.y, v.z, v.w};
    w0 = w1 = w2 = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int xi = int(rintf(ldexpf(vv[i], e)));  // |xi| <= 2^22
        const int c0 = (xi << 24) >> 24;              // balanced digits: c0, c1 in [-128, 127]
        const int r = (xi - c0) >> 8;
        const int c1 = (r << 24) >> 24;
        const int c2 = (r - c1) >> 8;                 // |c2| <= 64
        w0 |= uint32_t(c0 & 255) << (8 * i);
        w1 |= uint32_t(c1 & 255) << (8 * i);
        w2 |= uint32_t(c2 & 255) << (8 * i);
    }
    scale = ldexpf(1.f, -e);
}

// Stores the limbs of value word j of row `row` (from limbs4).
template <int T>
__device__ __forceinline__ void store_limbs(uint32_t *row, int K, int j, uint32_t w0, uint32_t w1, uint32_t w2,
                                            float scale) {
    const int lw = xq_lw(K), pj = lq_pad(j);
    row[pj] = w0;
    row[lw + pj] = w1;
    row[2 * lw + pj] = w2;
    if (j % kScaleWords<T> == 0) reinterpret_cast<float *>(row)[3 * lw + j / kScaleWords<T>] = scale;
}

// Workgroup-cooperative: rows [0, nb) of x [nb][ldx] (global, 16-byte aligned) to
// limbs in LDS.  Needs K % (4 kScaleWords) == 0; every thread must call it; the
// caller puts a barrier before the limbs are read.
template <int T>
__device__ __forceinline__ void stage_limbs(const float *x, int ldx, int nb, int K, uint32_t *lds) {
    const int nw = K >> 2, total = nb * nw, rw = xq_row_words<T>(K);
    for (int base = 0; base < total; base += blockDim.x) {
        // groups of kScaleWords lanes are all in or all out (total is a multiple)
        const int idx = base + int(threadIdx.x);
        const int jj = min(idx, total - 1);
        const int bi = jj / nw, j = jj - bi * nw;
        const float4 v = *reinterpret_cast<const float4 *>(x + size_t(bi) * ldx + 4 * j);
        uint32_t w0, w1, w2;
        float scale;
        limbs4<kScaleWords<T>>(v, w0, w1, w2, scale);
        if (idx < total) store_limbs<T>(lds + bi * rw, K, j, w0, w1, w2, scale);
    }
}

// This lane's chunks of the staged limb rows [0, nb) into registers (padding rows
// and chunks zero), with the per-chunk sums the dot products need.
template <int T, int B, int CPL>
__device__ __forceinline__ void gemv_load_xq(const uint32_t *lds, int K, int nb, const GemvGeom &g, int cl,
                                             XQ<T, B> (&xr)[CPL]) {
    constexpr int NW = XQ<T, B>::NW;
    const int lpr = 1 << g.lpr_log2, lw = xq_lw(K), rw = xq_row_words<T>(K);
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
        const int c = cl + t * lpr;
        const bool valid = c < g.nchunks;
        const int cc = valid ? c : 0;
        int run[NW / 4];  // value word of each 4-word run of the chunk
#pragma unroll
        for (int q = 0; q < NW / 4; ++q) {
            if constexpr (T == GGML_Q6_K) run[q] = (cc >> 2) * 64 + ((cc >> 1) & 1) * 32 + (cc & 1) * 4 + 8 * q;
            else if constexpr (T == GGML_Q8_0) run[q] = 8 * cc + 4 * q;
            else run[q] = (cc >> 2) * 64 + (cc & 3) * 16 + 4 * q;
        }
        const int sg = T == GGML_Q8_0 ? cc : (cc >> 2);
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            const bool v = valid && bi < nb;
            const uint32_t *row = lds + (bi < nb ? bi : 0) * rw;
#pragma unroll
            for (int l = 0; l < 3; ++l)
#pragma unroll
                for (int q = 0; q < NW / 4; ++q) {
                    const uint4 u = *reinterpret_cast<const uint4 *>(row + l * lw + lq_pad(run[q]));
                    xr[t].c[bi][l][4 * q] = v ? int(u.x) : 0;
                    xr[t].c[bi][l][4 * q + 1] = v ? int(u.y) : 0;
                    xr[t].c[bi][l][4 * q + 2] = v ? int(u.z) : 0;
                    xr[t].c[bi][l][4 * q + 3] = v ? int(u.w) : 0;
                }
            xr[t].sc[bi] = v ? reinterpret_cast<const float *>(row)[3 * lw + sg] : 0.f;
            if constexpr (T == GGML_Q4_K || T == GGML_Q5_K) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    int s3[3] = {0, 0, 0};
#pragma unroll
                    for (int l = 0; l < 3; ++l)
#pragma unroll
                        for (int u = 0; u < 8; ++u) s3[l] = sdot4(0x01010101u, xr[t].c[bi][l][8 * h + u], s3[l]);
                    xr[t].ms[bi][h] = xr[t].sc[bi] * limb_sum(s3[0], s3[1], s3[2]);
                }
            } else if constexpr (T == GGML_Q6_K) {
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int l = 0; l < 3; ++l) {
                        int s1 = 0;
#pragma unroll
                        for (int u = 0; u < 4; ++u) s1 = sdot4(0x01010101u, xr[t].c[bi][l][4 * q + u], s1);
                        xr[t].init[bi][q][l] = -32 * s1;
                    }
            }
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
// steps in flight).  G = 1 halves the arithmetic on a wave's critical path and the
// registers (every caller uses it); G = 2 keeps more bytes in flight per wave.
// Order of issue: pre() (loads the
// prologue needs, so that waiting for them does not wait for the weights: loads
// complete in order), the first step's weights, then prologue(), which fills
// xr and may use workgroup barriers (every thread of the workgroup must call
// this function).
// L2 > 0: g.lpr_log2 known at compile time (static lane-group reductions).
// DEPTH: steps of weights a wave keeps requested (2, or 3 for the long LM-head stream:
// more bytes in flight per wave at the same occupancy).
template <int T, int B, int CPL, bool NT = false, int G = 2, bool LM = false, int L2 = 0, int DEPTH = 2, class XR,
          class PreF, class Pro, class Epi>
__device__ __forceinline__ void gemv_rows(const WPtr &w, const GemvGeom &g, XR (&xr)[CPL], int gwave, int nwaves,
                                          PreF &&pre, Pro &&prologue, Epi &epi, const float *bias = nullptr,
                                          int nt_from = 0) {
    const int lane = threadIdx.x & 63;
    const int l2 = L2 > 0 ? L2 : g.lpr_log2;
    const int lpr = 1 << l2, rpw = 64 >> l2;
    const int grp = lane >> l2, cl = lane & (lpr - 1);
    int cidx[CPL];
#pragma unroll
    for (int t = 0; t < CPL; ++t) cidx[t] = (cl + t * lpr < g.nchunks) ? cl + t * lpr : 0;

    auto compute_step = [&](int rg, const Raw<T> (&r)[G][CPL], const float (&bv)[G]) {
#pragma unroll
        for (int u = 0; u < G; ++u) {
            float acc[B];
#pragma unroll
            for (int bi = 0; bi < B; ++bi) acc[bi] = 0.f;
#pragma unroll
            for (int t = 0; t < CPL; ++t) dot_chunk<T, B>(cidx[t], r[u][t], xr[t], acc);
#pragma unroll
            for (int bi = 0; bi < B; ++bi) {
                if constexpr (L2 > 0) acc[bi] = group_sum<1 << L2>(acc[bi]);
                else acc[bi] = group_sum_dyn(acc[bi], g.lpr_log2);
            }
            const int row = (rg + u * nwaves) * rpw + grp;
            if (cl == 0 && row < w.N) {
#pragma unroll
                for (int bi = 0; bi < B; ++bi) epi(row, bi, acc[bi] + bv[u]);
            }
        }
    };

    const int stride = G * nwaves;
    if constexpr (DEPTH > 2) {
        // step k of this wave: row group gwave + k stride, for k < nst.  Ring of DEPTH
        // buffers: the compute of step k is followed by the request of step k + DEPTH
        // into its buffer; the last DEPTH steps request nothing.  With NT, one cache
        // policy per wave (waves gwave < nt_from nwaves / N cached, the rest
        // non-temporal: the same share of rows as a row threshold); that choice and
        // whether there is a bias are made once, outside the loop, so that no load sits
        // behind a branch and every compute waits for its own step only.
        const int groups = (w.N + rpw - 1) / rpw;
        const int nst = gwave < groups ? (groups - gwave + stride - 1) / stride : 0;  // wave-uniform
        Raw<T> R[DEPTH][G][CPL];
        float bv[DEPTH][G];
        auto ring = [&](auto ntc, auto biasc) {
            constexpr bool NTW = decltype(ntc)::value, BIAS = decltype(biasc)::value;
            auto load = [&](int rg, Raw<T>(&r)[G][CPL], float(&b)[G]) {
#pragma unroll
                for (int u = 0; u < G; ++u) {
                    const int row = min((rg + u * nwaves) * rpw + grp, w.N - 1);
#pragma unroll
                    for (int t = 0; t < CPL; ++t) load_chunk<T, NTW, LM>(w, row, cidx[t], r[u][t]);
                    b[u] = BIAS ? bias[row] : 0.f;
                }
            };
            pre();
            __builtin_amdgcn_sched_barrier(0);
            static_for<0, DEPTH>([&](auto jc) {
                constexpr int j = decltype(jc)::value;
                if (j < nst) load(gwave + j * stride, R[j], bv[j]);
            });
            __builtin_amdgcn_sched_barrier(0);
            prologue();
            if (nst == 0) return;
            int k = 0;
            for (; k + 2 * DEPTH <= nst; k += DEPTH)  // every request of this round exists
                static_for<0, DEPTH>([&](auto jc) {
                    constexpr int j = decltype(jc)::value;
                    compute_step(gwave + (k + j) * stride, R[j], bv[j]);
                    load(gwave + (k + j + DEPTH) * stride, R[j], bv[j]);
                });
            static_for<0, DEPTH>([&](auto jc) {  // fewer than 2 DEPTH steps left
                constexpr int j = decltype(jc)::value;
                if (k + j < nst) {
                    compute_step(gwave + (k + j) * stride, R[j], bv[j]);
                    if (k + j + DEPTH < nst) load(gwave + (k + j + DEPTH) * stride, R[j], bv[j]);
                }
            });
            static_for<0, DEPTH>([&](auto jc) {
                constexpr int j = decltype(jc)::value;
                if (k + DEPTH + j < nst) compute_step(gwave + (k + DEPTH + j) * stride, R[j], bv[j]);
            });
        };
        using yes = std::integral_constant<bool, true>;
        using no = std::integral_constant<bool, false>;
        const bool ntw = NT && int64_t(gwave) * w.N >= int64_t(nt_from) * nwaves;  // wave-uniform
        if (ntw)
            bias ? ring(yes{}, yes{}) : ring(yes{}, no{});
        else
            bias ? ring(no{}, yes{}) : ring(no{}, no{});
        return;
    }
    // The choice of a bias is made once, outside the loop, and the first step is requested
    // by every wave (one past the last row group reads the last one and returns after
    // the prologue): a load behind a branch would leave the compiler unsure of the order
    // of the loads after it, and the prologue and each step would wait for all of them.
    auto run = [&](auto biasc) {
        constexpr bool BIAS = decltype(biasc)::value;
        auto load = [&](int rg, Raw<T>(&r)[G][CPL], float(&b)[G]) {
#pragma unroll
            for (int u = 0; u < G; ++u) {
                const int row = min((rg + u * nwaves) * rpw + grp, w.N - 1);
                if (NT && (rg + u * nwaves) * rpw >= nt_from) {  // wave-uniform
#pragma unroll
                    for (int t = 0; t < CPL; ++t) load_chunk<T, true, LM>(w, row, cidx[t], r[u][t]);
                } else {
#pragma unroll
                    for (int t = 0; t < CPL; ++t) load_chunk<T, false, LM>(w, row, cidx[t], r[u][t]);
                }
                b[u] = BIAS ? bias[row] : 0.f;
            }
        };
        int rg = gwave;
        const bool any = rg * rpw < w.N;  // wave-uniform
        Raw<T> A[G][CPL], Bf[G][CPL];
        float ba[G], bb[G];
        pre();
        __builtin_amdgcn_sched_barrier(0);
        load(min(rg, (w.N - 1) / rpw), A, ba);
        __builtin_amdgcn_sched_barrier(0);
        prologue();
        if (!any) return;
        // The last step is peeled off, so that every compute in the main loop follows
        // an issued prefetch: a conditional prefetch would merge two load states and
        // the compiler would wait for all loads (the prefetch included) before computing.
        for (;;) {
            const int rb = rg + stride;
            if (rb * rpw >= w.N) {  // wave-uniform
                compute_step(rg, A, ba);
                break;
            }
            load(rb, Bf, bb);
            compute_step(rg, A, ba);
            rg = rb;
            const int ra = rg + stride;
            if (ra * rpw >= w.N) {
                compute_step(rg, Bf, bb);
                break;
            }
            load(ra, A, ba);
            compute_step(rg, Bf, bb);
            rg = ra;
        }
    };
    if (bias)
        run(std::integral_constant<bool, true>{});
    else
        run(std::integral_constant<bool, false>{});
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
    return WPtr{w.q, w.s, w.d, w.N, w.K, w.K / ti.block_elems, w.tm};
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

// LDS bytes of nb staged limb rows of K values (0 for the f32-x formats)
inline size_t gemv_xq_lds(uint32_t t, int K, int nb) {
    switch (t) {
    case GGML_Q4_K: return xq_lds_bytes<GGML_Q4_K>(K, nb);
    case GGML_Q5_K: return xq_lds_bytes<GGML_Q5_K>(K, nb);
    case GGML_Q6_K: return xq_lds_bytes<GGML_Q6_K>(K, nb);
    case GGML_Q8_0: return xq_lds_bytes<GGML_Q8_0>(K, nb);
    default: return 0;
    }
}

}  // namespace mlg
