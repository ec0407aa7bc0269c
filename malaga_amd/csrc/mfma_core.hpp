// MFMA operands from quantized weights (gfx950 f16 MFMA), shared by the GEMM kernels:
// the integer quants (q4_K / q5_K nibbles, q6_K 6-bit values - 32, q8_0 int8) are exact
// in f16, so they are the B operand as they are; block scales and k-quant mins are
// applied per sub-block in f32 by the caller:
//   sum_k w_k x_k = d sc * sum_k q_k x_k - dmin m * sum_k x_k,
// or folded into B where that stays exact (FOLD: q4_K / q5_K in the decode GEMMs;
// SPLIT: q6_K as an exact f16 pair in the prefill / LM-head GEMMs).
// B-operand layout (16x16x32 / 16x16x16 f16 MFMA): lane l holds W row l % 16 and the
// k-group l / 16 of the sub-block.  Quant bytes become f16 with v_perm
// (byte -> 0x64xx = 1024 + byte) and one packed f16 subtraction.
#pragma once
#include "device.hpp"
#include "gemv_core.hpp"

namespace mlg {


constexpr int kStep = 256;  // K per W fetch (one k-quant super-block)


// f16 pair (1024 + byte sel0, 1024 + byte sel1) of v, minus `off` (exact for bytes < 1024 - off range)
__device__ __forceinline__ uint32_t bytes_to_h2(uint32_t v, uint32_t sel, h2_t off) {
    const uint32_t p = __builtin_amdgcn_perm(0x64646464u, v, sel);
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, p) - off);
}
// the 4 bytes of v as 4 f16 values (byte - (off - 1024)) in natural order
__device__ __forceinline__ uint2 bytes_to_h4(uint32_t v, h2_t off) {
    return make_uint2(bytes_to_h2(v, 0x04010400u, off), bytes_to_h2(v, 0x04030402u, off));
}

template <int T>
struct MW;  // per-type W fetch for one 256-wide K step

// Scale folding (FOLD types, q4_K / q5_K): the 6-bit sub-block scale a_s times a quant
// (q <= 15, or 31 for q5_K) is at most 1953, an exact f16 integer, so B = a_s q is the MFMA
// operand and the 8 slices of a block accumulate in the MFMA's own C operand; the min term
// sum_k m_s x_k also runs on the MFMA (B = m_s in every element).  Per block then
//   sum_k w_k x_k = d C - dmin M,   C = sum_s X_s (a_s q_s),   M = sum_s X_s m_s,
// instead of two f32 FMAs per output and slice.
//
// The 8 sub-block scales and mins of a block are decoded once per block (fold_prep) as f16
// pairs: pair i holds sub-blocks 2 i and 2 i + 1, and na = -1024 a.  q4_K then builds B with
// one packed FMA per pair of values, fma(1024 + q, a, -1024 a) = q a: v_perm gives 1024 + q
// exactly, (1024 + 15) * 63 <= 65504 stays finite, and the result q a <= 945 is exact.
// q5_K (q <= 31 would overflow that product) subtracts 1024 first and then multiplies.
struct FoldPrep {
    uint32_t a[4], na[4], m[4];
};
// the k-quant header's 6-bit scales a_j and mins m_j (j < 8, get_scale_min_k4 in ggml's
// k-quants) for all 8 sub-blocks at once, bytewise: j < 4 from the low 6 bits of bytes j,
// j + 4; j >= 4 from the nibbles of byte j + 4 and the top 2 bits of bytes j - 4, j
__device__ __forceinline__ FoldPrep k4_fold_prep(const uint4 &hdr) {
    const uint32_t a03 = hdr.y & 0x3F3F3F3Fu, m03 = hdr.z & 0x3F3F3F3Fu;
    const uint32_t a47 = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
    const uint32_t m47 = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
    const h2_t off = {_Float16(1024), _Float16(1024)}, neg = {_Float16(-1024), _Float16(-1024)};
    const uint2 a0 = bytes_to_h4(a03, off), a1 = bytes_to_h4(a47, off);
    const uint2 m0 = bytes_to_h4(m03, off), m1 = bytes_to_h4(m47, off);
    FoldPrep p;
    p.a[0] = a0.x, p.a[1] = a0.y, p.a[2] = a1.x, p.a[3] = a1.y;
    p.m[0] = m0.x, p.m[1] = m0.y, p.m[2] = m1.x, p.m[3] = m1.y;
#pragma unroll
    for (int i = 0; i < 4; ++i) p.na[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, p.a[i]) * neg);
    return p;
}
// half h of the f16 pair u in both halves
__device__ __forceinline__ h2_t splat_half(uint32_t u, int h) {
    const h2_t v = __builtin_bit_cast(h2_t, u);
    return h ? __builtin_shufflevector(v, v, 1, 1) : __builtin_shufflevector(v, v, 0, 0);
}

template <class W>
__device__ __forceinline__ FoldPrep fold_prep(const typename W::Regs &r) {
    return k4_fold_prep(r.hdr);
}

template <class W>
__device__ __forceinline__ void fold_slice(const typename W::Regs &r, const FoldPrep &p, int s, const h8_t &ah,
                                           const h8_t &al, f4_t &cb, f4_t &mb) {
    const h8_t bq = W::b_fold(r, p, s);
    const h2_t m2 = splat_half(p.m[s >> 1], s & 1);
    const h8_t bm = __builtin_shufflevector(m2, m2, 0, 1, 0, 1, 0, 1, 0, 1);
    cb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq, cb, 0, 0, 0);
    cb = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq, cb, 0, 0, 0);
    mb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bm, mb, 0, 0, 0);
    mb = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bm, mb, 0, 0, 0);
}
// acc += d C - dmin M at the end of a block (live false: a block past the end weighs 0)
template <class W>
__device__ __forceinline__ void fold_flush(const typename W::Regs &r, bool live, const f4_t &cb, const f4_t &mb,
                                           f4_t &acc) {
    const float d = live ? h2f(r.hdr.x) : 0.f, dmin = live ? h2f(r.hdr.x >> 16) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = fmaf(d, cb[i], fmaf(-dmin, mb[i], acc[i]));
}

// q4_K: 8 sub-blocks of 32; lane k-group kq reads bytes qs[32 g + 8 kq, +8) of the
// 4 byte groups g (low nibbles: sub-block 2g, high nibbles: 2g + 1).
template <>
struct MW<GGML_Q4_K> {
    static constexpr int SLICES = 8, SK = 32;
    static constexpr bool MIN = true;  // w = sc q - mn: the x sums carry the min term
    struct Regs {
        uint4 hdr;
        uint2 q[4];
    };
    __device__ static void load(const WPtr &w, int row, int kb, int kq, Regs &r) {
        const uint8_t *blk = w.q + (size_t(row) * w.nb + kb) * 144;
        r.hdr = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
        for (int g = 0; g < 4; ++g) r.q[g] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * g + 8 * kq);
    }
    // the same registers from the tile-major copy (kQ4TileBytes per tile and block)
    __device__ static void load_tile(const uint8_t *tw, int nb, int tile, int kb, int kq, int ln, Regs &r) {
        const uint8_t *tb = tw + (size_t(tile) * nb + kb) * kQ4TileBytes;
        const int li = 16 * kq + ln;
        r.hdr = *reinterpret_cast<const uint4 *>(tb + 16 * ln);
        const uint4 a = *reinterpret_cast<const uint4 *>(tb + 256 + 16 * li);
        const uint4 b = *reinterpret_cast<const uint4 *>(tb + 1280 + 16 * li);
        r.q[0] = make_uint2(a.x, a.y), r.q[1] = make_uint2(a.z, a.w);
        r.q[2] = make_uint2(b.x, b.y), r.q[3] = make_uint2(b.z, b.w);
    }
    __device__ static h8_t b(const Regs &r, int s) {
        const uint2 q = r.q[s >> 1];
        const int sh = 4 * (s & 1);
        const h2_t off = {_Float16(1024), _Float16(1024)};
        const uint2 lo = bytes_to_h4((q.x >> sh) & 0x0F0F0F0Fu, off), hi = bytes_to_h4((q.y >> sh) & 0x0F0F0F0Fu, off);
        return __builtin_bit_cast(h8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
    }
    __device__ static void scale(const Regs &r, int s, float &sc, float &mn) {
        float a, m;
        k4_scale_min(s, r.hdr.y, r.hdr.z, r.hdr.w, a, m);
        sc = h2f(r.hdr.x) * a;
        mn = h2f(r.hdr.x >> 16) * m;
    }
    static constexpr bool FOLD = true;
    static constexpr bool SPLIT = false;
    // B = a_s q of slice s (FoldPrep): v_perm's 1024 + q times a_s, minus 1024 a_s, in one FMA
    __device__ static h8_t b_fold(const Regs &r, const FoldPrep &p, int s) {
        const uint2 q = r.q[s >> 1];
        const int sh = 4 * (s & 1);
        const uint32_t v0 = (q.x >> sh) & 0x0F0F0F0Fu, v1 = (q.y >> sh) & 0x0F0F0F0Fu;
        const h2_t a = splat_half(p.a[s >> 1], s & 1), na = splat_half(p.na[s >> 1], s & 1);
        auto pair = [&](uint32_t v, uint32_t sel) {
            const h2_t raw = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, v, sel));
            return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(raw, a, na));
        };
        return __builtin_bit_cast(h8_t, make_uint4(pair(v0, 0x04010400u), pair(v0, 0x04030402u), pair(v1, 0x04010400u),
                                                   pair(v1, 0x04030402u)));
    }
};

// q5_K: as q4_K plus the fifth bit of sub-block s in bit s of qh[l] (l < 32).
template <>
struct MW<GGML_Q5_K> {
    static constexpr int SLICES = 8, SK = 32;
    static constexpr bool MIN = true;
    struct Regs {
        uint4 hdr;
        uint2 q[4];
        uint2 qh;
    };
    __device__ static void load(const WPtr &w, int row, int kb, int kq, Regs &r) {
        const uint8_t *blk = w.q + (size_t(row) * w.nb + kb) * 176;
        r.hdr = *reinterpret_cast<const uint4 *>(blk);
        r.qh = *reinterpret_cast<const uint2 *>(blk + 16 + 8 * kq);
#pragma unroll
        for (int g = 0; g < 4; ++g) r.q[g] = *reinterpret_cast<const uint2 *>(blk + 48 + 32 * g + 8 * kq);
    }
    __device__ static h8_t b(const Regs &r, int s) {
        const uint2 q = r.q[s >> 1];
        const int sh = 4 * (s & 1);
        const h2_t off = {_Float16(1024), _Float16(1024)};
        const uint32_t v0 = ((q.x >> sh) & 0x0F0F0F0Fu) | (((r.qh.x >> s) & 0x01010101u) << 4);
        const uint32_t v1 = ((q.y >> sh) & 0x0F0F0F0Fu) | (((r.qh.y >> s) & 0x01010101u) << 4);
        const uint2 lo = bytes_to_h4(v0, off), hi = bytes_to_h4(v1, off);
        return __builtin_bit_cast(h8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
    }
    __device__ static void scale(const Regs &r, int s, float &sc, float &mn) {
        MW<GGML_Q4_K>::Regs t{r.hdr, {}};
        MW<GGML_Q4_K>::scale(t, s, sc, mn);
    }
    static constexpr bool FOLD = true;
    static constexpr bool SPLIT = false;
    // B = a_s q (q <= 31: (1024 + q) a_s could exceed the f16 range, so q first)
    __device__ static h8_t b_fold(const Regs &r, const FoldPrep &p, int s) {
        const h2_t a = splat_half(p.a[s >> 1], s & 1);
        const h8_t av = __builtin_shufflevector(a, a, 0, 1, 0, 1, 0, 1, 0, 1);
        return b(r, s) * av;
    }
};

// q6_K: 16 groups of 16 with an int8 scale each (one 16x16x16 MFMA per group).
// Group G = 8 n + 2 t + h holds values 128 n + 32 t + 16 h + j (j < 16): low 4 bits
// from ql[64 n + 32 (t & 1) + 16 h + j] (nibble t >> 1), high 2 bits from
// qh[32 n + 16 h + j] bits 2t..2t+1.  Lane k-group kq takes j = 4 kq .. 4 kq + 3.
template <>
struct MW<GGML_Q6_K> {
    static constexpr int SLICES = 16, SK = 16;
    static constexpr bool MIN = false;
    static constexpr bool FOLD = false;
    struct Regs {
        uint32_t qa[4], qb[4], qh[4];  // [2 n + h]
        uint4 sc;
        // 16 bits as loaded: a 32-bit field would be zero-extended right after the load,
        // which makes the wave wait for its prefetched block before computing this one
        unsigned short d;
    };
    __device__ static void load(const WPtr &w, int row, int kb, int kq, Regs &r) {
        const size_t blk = size_t(row) * w.nb + kb;
        const uint8_t *qp = w.q + blk * 192;
#pragma unroll
        for (int nh = 0; nh < 4; ++nh) {
            const int n = nh >> 1, h = nh & 1;
            r.qa[nh] = *reinterpret_cast<const uint32_t *>(qp + 64 * n + 16 * h + 4 * kq);
            r.qb[nh] = *reinterpret_cast<const uint32_t *>(qp + 64 * n + 32 + 16 * h + 4 * kq);
            r.qh[nh] = *reinterpret_cast<const uint32_t *>(qp + 128 + 32 * n + 16 * h + 4 * kq);
        }
        r.sc = *reinterpret_cast<const uint4 *>(w.s + blk * 16);
        r.d = *reinterpret_cast<const unsigned short *>(w.d + blk * 2);
    }
    // the same registers from the tile-major copy (kQ6TileBytes per tile and block):
    // five loads, each of whole cache lines, instead of fourteen of 16 scattered rows
    __device__ static void load_tile(const uint8_t *tw, int nb, int tile, int kb, int kq, int ln, Regs &r) {
        const uint8_t *tb = tw + (size_t(tile) * nb + kb) * kQ6TileBytes;
        const int li = 16 * kq + ln;
        const uint4 a = *reinterpret_cast<const uint4 *>(tb + 16 * li);
        const uint4 b = *reinterpret_cast<const uint4 *>(tb + 1024 + 16 * li);
        const uint4 h = *reinterpret_cast<const uint4 *>(tb + 2048 + 16 * li);
        r.qa[0] = a.x, r.qa[1] = a.y, r.qa[2] = a.z, r.qa[3] = a.w;
        r.qb[0] = b.x, r.qb[1] = b.y, r.qb[2] = b.z, r.qb[3] = b.w;
        r.qh[0] = h.x, r.qh[1] = h.y, r.qh[2] = h.z, r.qh[3] = h.w;
        r.sc = *reinterpret_cast<const uint4 *>(tb + 3072 + 16 * ln);
        r.d = *reinterpret_cast<const unsigned short *>(tb + 3328 + 2 * ln);
    }
    __device__ static h4_t b(const Regs &r, int G) {
        const int n = G >> 3, t = (G >> 1) & 3, h = G & 1, nh = 2 * n + h;
        const uint32_t ql = (t & 1) ? r.qb[nh] : r.qa[nh];
        const uint32_t v = ((ql >> (4 * (t >> 1))) & 0x0F0F0F0Fu) | (((r.qh[nh] >> (2 * t)) & 0x03030303u) << 4);
        const h2_t off = {_Float16(1056), _Float16(1056)};  // 1024 + 32
        return __builtin_bit_cast(h4_t, bytes_to_h4(v, off));
    }
    __device__ static void scale(const Regs &r, int G, float &sc, float &mn) {
        const uint32_t wv = G < 8 ? (G < 4 ? r.sc.x : r.sc.y) : (G < 12 ? r.sc.z : r.sc.w);
        sc = h2f(r.d) * float(int8_t(wv >> (8 * (G & 3))));
        mn = 0.f;
    }
    // Split-B slices (SPLIT): the 16x16x32 MFMA over the two groups 2 s and 2 s + 1 of
    // 32-slice s, with the int8 group scale folded into B.  |q sc| <= 32 * 128 = 4096 is
    // an integer, so bh = f16(q sc) (one rounding) and bl = q sc - bh (in {-1, 0, 1}) are
    // exact and sum to q sc; with x = xh + xl the product is xh bh + xl bh + xh bl up to
    // xl bl (<= 2^-22 |x q sc|).  The lane keeps its registers: elements 0..3 are
    // j = 4 kq .. 4 kq + 3 of group 2 s, elements 4..7 the same j of group 2 s + 1, so the
    // A fragment of lane k-group kq is x[32 s + 4 kq + e] then x[32 s + 16 + 4 kq + e]
    // (split_pos gives where the staged X keeps them).  Per block then
    //   sum_k w_k x_k = d C,   C = sum_s (xh bh_s + xl bh_s + xh bl_s)   (MFMA C operand).
    static constexpr bool SPLIT = true;
    static constexpr int SLICES32 = 8;
    __device__ static void b_split(const Regs &r, int s, h8_t &bh, h8_t &bl) {
        const h4_t q0 = b(r, 2 * s), q1 = b(r, 2 * s + 1);
        const uint32_t wv = s < 4 ? (s < 2 ? r.sc.x : r.sc.y) : (s < 6 ? r.sc.z : r.sc.w);
        const int sh = 16 * (s & 1);
        const _Float16 f0 = _Float16(float(int8_t(wv >> sh))), f1 = _Float16(float(int8_t(wv >> (sh + 8))));
        const h8_t q = {q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
        const h8_t sc = {f0, f0, f0, f0, f1, f1, f1, f1};
        bh = q * sc;
        bl = __builtin_elementwise_fma(q, sc, -bh);
    }
    __device__ static float d_of(const Regs &r) { return h2f(r.d); }
};

// Position in the staged X of the 4-value group g4 (0..7) of a 32-slice for split-B
// slices: group g4 < 4 sits at 2 g4, group 4 + g at 2 g + 1, so lane k-group kq reads
// its A fragment (groups kq and 4 + kq) as the 8 halves at 8 kq.
__host__ __device__ constexpr int split_pos(int g4) { return g4 < 4 ? 2 * g4 : 2 * (g4 - 4) + 1; }

// q8_0: 8 blocks of 32 per step, int8 values (q ^ 0x80 = q + 128 as a byte).
template <>
struct MW<GGML_Q8_0> {
    static constexpr int SLICES = 8, SK = 32;
    static constexpr bool MIN = false;
    static constexpr bool FOLD = false;
    static constexpr bool SPLIT = false;
    struct Regs {
        uint2 q[8];
        uint4 d;  // 8 f16 scales
    };
    __device__ static void load(const WPtr &w, int row, int kb, int kq, Regs &r) {
        const uint8_t *qp = w.q + size_t(row) * w.K + size_t(kb) * 256 + 8 * kq;
#pragma unroll
        for (int b = 0; b < 8; ++b) r.q[b] = *reinterpret_cast<const uint2 *>(qp + 32 * b);
        r.d = *reinterpret_cast<const uint4 *>(w.d + (size_t(row) * (w.K >> 5) + size_t(kb) * 8) * 2);
    }
    __device__ static h8_t b(const Regs &r, int s) {
        const h2_t off = {_Float16(1152), _Float16(1152)};  // 1024 + 128
        const uint2 lo = bytes_to_h4(r.q[s].x ^ 0x80808080u, off), hi = bytes_to_h4(r.q[s].y ^ 0x80808080u, off);
        return __builtin_bit_cast(h8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
    }
    __device__ static void scale(const Regs &r, int s, float &sc, float &mn) {
        const uint32_t wv = s < 4 ? (s < 2 ? r.d.x : r.d.y) : (s < 6 ? r.d.z : r.d.w);
        sc = h2f(wv >> (16 * (s & 1)));
        mn = 0.f;
    }
};

// f16 weights: used as they are.
template <>
struct MW<GGML_F16> {
    static constexpr int SLICES = 8, SK = 32;
    static constexpr bool MIN = false;
    static constexpr bool FOLD = false;
    static constexpr bool SPLIT = false;
    struct Regs {
        uint4 q[8];
    };
    __device__ static void load(const WPtr &w, int row, int kb, int kq, Regs &r) {
        const uint8_t *qp = w.q + (size_t(row) * w.K + size_t(kb) * 256 + 8 * kq) * 2;
#pragma unroll
        for (int s = 0; s < 8; ++s) r.q[s] = *reinterpret_cast<const uint4 *>(qp + 64 * s);
    }
    __device__ static h8_t b(const Regs &r, int s) { return __builtin_bit_cast(h8_t, r.q[s]); }
    __device__ static void scale(const Regs &, int, float &sc, float &mn) {
        sc = 1.f;
        mn = 0.f;
    }
};

// W registers of row 16 tile + ln, K block kb: from the tile-major copy (TL, q6_K / q4_K; a
// tile past the last reads the last) or from the planes (the row clamped to N - 1)
template <int T, bool TL>
__device__ __forceinline__ void load_w(const WPtr &w, int tile, int ln, int kb, int kq, typename MW<T>::Regs &r) {
    if constexpr (TL) MW<T>::load_tile(w.t, w.nb, min(tile, (w.N + 15) / 16 - 1), kb, kq, ln, r);
    else MW<T>::load(w, min(16 * tile + ln, w.N - 1), kb, kq, r);
}

}  // namespace mlg
