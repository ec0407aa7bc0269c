// Dequant-GEMV for decode (batch 1..4): y[b][n] = sum_k x[b][k] * W[n][k].
//
// Work layout (wave64): each lane owns a fixed "chunk" of the row (a k-range of
// XW weights) for the whole kernel, so its slice of x stays in registers; the
// lanes of a row group (LPR lanes, a power of two) stream one row with 16-byte
// loads, and a wave covers 64/LPR rows per step.  Waves stride over rows and
// handle two row groups per iteration to keep more loads in flight.  Integer
// quants are widened with v_cvt_f32_ubyte* and accumulated in f32; block
// offsets (q4_K/q5_K min, q6_K -32, q8_0 sign) are applied once per group from
// per-lane x sums, so the inner loop is mask + convert + FMA.
#include "device.hpp"
#include "kernels.hpp"
#include "quant.hpp"

namespace mlg {

namespace {

template <int T>
struct Traits;
template <>
struct Traits<GGML_Q4_K> { static constexpr int XW = 64, NS = 2; };  // chunk = 64-weight group g
template <>
struct Traits<GGML_Q5_K> { static constexpr int XW = 64, NS = 2; };
template <>
struct Traits<GGML_Q6_K> { static constexpr int XW = 64, NS = 4; };  // chunk = (half, 16-lane) slice
template <>
struct Traits<GGML_Q8_0> { static constexpr int XW = 32, NS = 1; };  // chunk = one block
template <>
struct Traits<GGML_F16> { static constexpr int XW = 8, NS = 1; };
template <>
struct Traits<GGML_F32> { static constexpr int XW = 4, NS = 1; };

struct GemvParams {
    const uint8_t *q, *s, *d;
    const float *x;
    int ldx;
    float *y;
    int ldy;
    const float *bias;
    int relu;
    int N, K, nb;     // nb: blocks per row
    int lpr_log2;     // lanes per row group = 1 << lpr_log2 (<= 64)
    int nchunks;      // chunks per row
    int b;            // valid batch rows
    float *pv;        // argmax partials [b][gridDim.x]
    uint32_t *pi;
    int mask_id;
};

// x position of element e (0..XW-1) of chunk c
template <int T>
__device__ __forceinline__ int xpos(int c, int e) {
    if constexpr (T == GGML_Q4_K || T == GGML_Q5_K) {
        return (c >> 2) * 256 + (c & 3) * 64 + e;
    } else if constexpr (T == GGML_Q6_K) {
        const int j = c >> 2, h2 = (c >> 1) & 1, i = c & 1;
        return j * 256 + h2 * 128 + i * 16 + (e >> 4) * 32 + (e & 15);
    } else {
        return c * Traits<T>::XW + e;
    }
}

// x sum slot of element e
template <int T>
__device__ __forceinline__ int xslot(int e) {
    if constexpr (T == GGML_Q4_K || T == GGML_Q5_K) return e >> 5;
    else if constexpr (T == GGML_Q6_K) return e >> 4;
    else return 0;
}

// Raw bytes of one chunk of one row.
template <int T>
struct Raw {
    uint4 a, b, c, h, e;
    uint32_t e0, e1;
};

template <int T>
__device__ __forceinline__ void load_chunk(const GemvParams &p, int row, int c, Raw<T> &r) {
    if constexpr (T == GGML_Q4_K) {
        const uint8_t *blk = p.q + (size_t(row) * p.nb + (c >> 2)) * 144;
        const int g = c & 3;
        r.h = *reinterpret_cast<const uint4 *>(blk);
        r.a = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * g);
        r.b = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * g);
    } else if constexpr (T == GGML_Q5_K) {
        const uint8_t *blk = p.q + (size_t(row) * p.nb + (c >> 2)) * 176;
        const int g = c & 3;
        r.h = *reinterpret_cast<const uint4 *>(blk);
        r.c = *reinterpret_cast<const uint4 *>(blk + 16);  // qh[0..15]
        r.e = *reinterpret_cast<const uint4 *>(blk + 32);  // qh[16..31]
        r.a = *reinterpret_cast<const uint4 *>(blk + 48 + 32 * g);
        r.b = *reinterpret_cast<const uint4 *>(blk + 64 + 32 * g);
    } else if constexpr (T == GGML_Q6_K) {
        const size_t blk = size_t(row) * p.nb + (c >> 2);
        const int h2 = (c >> 1) & 1, i = c & 1;
        const uint8_t *qp = p.q + blk * 192;
        r.a = *reinterpret_cast<const uint4 *>(qp + 64 * h2 + 16 * i);
        r.b = *reinterpret_cast<const uint4 *>(qp + 64 * h2 + 32 + 16 * i);
        r.h = *reinterpret_cast<const uint4 *>(qp + 128 + 32 * h2 + 16 * i);
        const uint2 sc = *reinterpret_cast<const uint2 *>(p.s + blk * 16 + 8 * h2);
        r.e0 = sc.x;
        r.e1 = sc.y;
        r.c.x = *reinterpret_cast<const unsigned short *>(p.d + blk * 2);
    } else if constexpr (T == GGML_Q8_0) {
        const uint8_t *qp = p.q + size_t(row) * p.K + 32 * c;
        r.a = *reinterpret_cast<const uint4 *>(qp);
        r.b = *reinterpret_cast<const uint4 *>(qp + 16);
        r.e0 = *reinterpret_cast<const unsigned short *>(p.d + (size_t(row) * (p.K >> 5) + c) * 2);
    } else if constexpr (T == GGML_F16) {
        r.a = *reinterpret_cast<const uint4 *>(p.q + (size_t(row) * p.K + 8 * c) * 2);
    } else {
        r.a = *reinterpret_cast<const uint4 *>(p.q + (size_t(row) * p.K + 4 * c) * 4);
    }
}

template <int T, int B>
__device__ __forceinline__ void dot_chunk(const GemvParams &p, int row, int c, const Raw<T> &r,
                                          const float (&x)[B][Traits<T>::XW], const float (&xs)[B][Traits<T>::NS],
                                          float (&acc)[B]) {
    if constexpr (T == GGML_Q4_K || T == GGML_Q5_K) {
        const int g = c & 3;
        // scale/min of sub-blocks 2g (low nibbles) and 2g+1 (high nibbles)
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
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            float al = 0.f, ah = 0.f;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                uint32_t lo, hi;
                if constexpr (T == GGML_Q5_K) {
                    lo = (w[u] & 0x0F0F0F0Fu) | (((hb[u] >> (2 * g)) & 0x01010101u) << 4);
                    hi = ((w[u] >> 4) & 0x0F0F0F0Fu) | (((hb[u] >> (2 * g + 1)) & 0x01010101u) << 4);
                } else {
                    lo = w[u] & 0x0F0F0F0Fu;
                    hi = w[u] & 0xF0F0F0F0u;  // 16 * nibble; scaled back below
                }
                al = dot4u8(lo, &x[bi][4 * u], al);
                ah = dot4u8(hi, &x[bi][32 + 4 * u], ah);
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
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t g0 = (A[u] & 0x0F0F0F0Fu) | ((H[u] << 4) & 0x30303030u);
                const uint32_t g1 = (Bq[u] & 0x0F0F0F0Fu) | ((H[u] << 2) & 0x30303030u);
                const uint32_t g2 = ((A[u] >> 4) & 0x0F0F0F0Fu) | (H[u] & 0x30303030u);
                const uint32_t g3 = ((Bq[u] >> 4) & 0x0F0F0F0Fu) | ((H[u] >> 2) & 0x30303030u);
                a0 = dot4u8(g0, &x[bi][4 * u], a0);
                a1 = dot4u8(g1, &x[bi][16 + 4 * u], a1);
                a2 = dot4u8(g2, &x[bi][32 + 4 * u], a2);
                a3 = dot4u8(g3, &x[bi][48 + 4 * u], a3);
            }
            acc[bi] += d * (sc[0] * (a0 - 32.f * xs[bi][0]) + sc[1] * (a1 - 32.f * xs[bi][1]) +
                            sc[2] * (a2 - 32.f * xs[bi][2]) + sc[3] * (a3 - 32.f * xs[bi][3]));
        }
    } else if constexpr (T == GGML_Q8_0) {
        const float d = h2f(r.e0);
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            float a = 0.f;
#pragma unroll
            for (int u = 0; u < 8; ++u) a = dot4u8(w[u] ^ 0x80808080u, &x[bi][4 * u], a);  // q + 128
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

template <int T, int B, int CPL, int MODE>
__global__ __launch_bounds__(256) void k_gemv(GemvParams p) {
    constexpr int XW = Traits<T>::XW, NS = Traits<T>::NS;
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << p.lpr_log2, rpw = 64 >> p.lpr_log2;
    const int grp = lane >> p.lpr_log2, cl = lane & (lpr - 1);
    const int gwave = blockIdx.x * 4 + (threadIdx.x >> 6), nwaves = gridDim.x * 4;

    float x[CPL][B][XW];
    float xs[CPL][B][NS];
    bool cval[CPL];
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
        const int c = cl + t * lpr;
        cval[t] = c < p.nchunks;
        const int cc = cval[t] ? c : 0;
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
#pragma unroll
            for (int s = 0; s < NS; ++s) xs[t][bi][s] = 0.f;
#pragma unroll
            for (int e = 0; e < XW; ++e) {
                const float v = (bi < p.b && cval[t]) ? p.x[size_t(bi) * p.ldx + xpos<T>(cc, e)] : 0.f;
                x[t][bi][e] = v;
                xs[t][bi][xslot<T>(e)] += v;
            }
        }
    }

    float best[B];
    uint32_t bidx[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi) {
        best[bi] = -INFINITY;
        bidx[bi] = 0xffffffffu;
    }

    for (int rg = gwave; rg * rpw < p.N; rg += 2 * nwaves) {
        const int row0 = rg * rpw + grp, row1 = (rg + nwaves) * rpw + grp;
        const int r0 = min(row0, p.N - 1), r1 = min(row1, p.N - 1);
        Raw<T> w0[CPL], w1[CPL];
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            const int c = cval[t] ? cl + t * lpr : 0;
            load_chunk<T>(p, r0, c, w0[t]);
            load_chunk<T>(p, r1, c, w1[t]);
        }
        float acc0[B], acc1[B];
#pragma unroll
        for (int bi = 0; bi < B; ++bi) acc0[bi] = acc1[bi] = 0.f;
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            if (cval[t]) {
                const int c = cl + t * lpr;
                dot_chunk<T, B>(p, r0, c, w0[t], x[t], xs[t], acc0);
                dot_chunk<T, B>(p, r1, c, w1[t], x[t], xs[t], acc1);
            }
        }
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            for (int o = lpr >> 1; o > 0; o >>= 1) {
                acc0[bi] += __shfl_xor(acc0[bi], o, 64);
                acc1[bi] += __shfl_xor(acc1[bi], o, 64);
            }
        }
        if (cl == 0) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int row = h ? row1 : row0;
                if (row >= p.N) continue;
#pragma unroll
                for (int bi = 0; bi < B; ++bi) {
                    if (bi >= p.b) continue;
                    float v = h ? acc1[bi] : acc0[bi];
                    if (p.bias) v += p.bias[row];
                    if constexpr (MODE == 0) {
                        if (p.relu) v = fmaxf(v, 0.f);
                        p.y[size_t(bi) * p.ldy + row] = v;
                    } else {
                        if (row != p.mask_id) argmax_merge(best[bi], bidx[bi], v, uint32_t(row));
                    }
                }
            }
        }
    }

    if constexpr (MODE == 1) {
        __shared__ float sv[4][B];
        __shared__ uint32_t si[4][B];
        const int w = threadIdx.x >> 6;
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            wave_argmax(best[bi], bidx[bi]);
            if (lane == 0) {
                sv[w][bi] = best[bi];
                si[w][bi] = bidx[bi];
            }
        }
        __syncthreads();
        if (threadIdx.x < B && int(threadIdx.x) < p.b) {
            const int bi = threadIdx.x;
            float v = sv[0][bi];
            uint32_t i = si[0][bi];
            for (int k = 1; k < 4; ++k) argmax_merge(v, i, sv[k][bi], si[k][bi]);
            p.pv[size_t(bi) * gridDim.x + blockIdx.x] = v;
            p.pi[size_t(bi) * gridDim.x + blockIdx.x] = i;
        }
    }
}

int xw_of(uint32_t t) {
    switch (t) {
    case GGML_Q4_K: case GGML_Q5_K: case GGML_Q6_K: return 64;
    case GGML_Q8_0: return 32;
    case GGML_F16: return 8;
    case GGML_F32: return 4;
    default: return 0;
    }
}

// lanes per row group and chunks per lane for matrix w
bool geometry(const DevMatrix &w, int *lpr_log2, int *cpl, int *nchunks) {
    const int xw = xw_of(w.type);
    if (!xw || w.K % xw) return false;
    const int nc = w.K / xw;
    int l2 = 0;
    while ((1 << l2) < nc && l2 < 6) ++l2;
    *lpr_log2 = l2;
    *cpl = (nc + 63) / 64;
    *nchunks = nc;
    return *cpl <= 4;
}

constexpr int kMaxXRegs = 128;

template <int T, int B, int CPL, int MODE>
hipError_t launch_t(const GemvParams &p, int grid, hipStream_t st) {
    if constexpr (Traits<T>::XW * B * CPL > kMaxXRegs) {
        return hipErrorInvalidValue;
    } else {
        hipLaunchKernelGGL((k_gemv<T, B, CPL, MODE>), dim3(grid), dim3(256), 0, st, p);
        return hipGetLastError();
    }
}

template <int T, int MODE>
hipError_t dispatch_bc(const GemvParams &p, int B, int cpl, int grid, hipStream_t st) {
#define MLG_CASE(BB, CC) \
    if (B == BB && cpl == CC) return launch_t<T, BB, CC, MODE>(p, grid, st);
    MLG_CASE(1, 1) MLG_CASE(1, 2) MLG_CASE(1, 4)
    MLG_CASE(2, 1) MLG_CASE(2, 2) MLG_CASE(2, 4)
    MLG_CASE(4, 1) MLG_CASE(4, 2) MLG_CASE(4, 4)
#undef MLG_CASE
    return hipErrorInvalidValue;
}

template <int MODE>
hipError_t dispatch(const DevMatrix &w, const GemvParams &p, int B, int cpl, int grid, hipStream_t st) {
    switch (w.type) {
    case GGML_Q4_K: return dispatch_bc<GGML_Q4_K, MODE>(p, B, cpl, grid, st);
    case GGML_Q5_K: return dispatch_bc<GGML_Q5_K, MODE>(p, B, cpl, grid, st);
    case GGML_Q6_K: return dispatch_bc<GGML_Q6_K, MODE>(p, B, cpl, grid, st);
    case GGML_Q8_0: return dispatch_bc<GGML_Q8_0, MODE>(p, B, cpl, grid, st);
    case GGML_F16: return dispatch_bc<GGML_F16, MODE>(p, B, cpl, grid, st);
    case GGML_F32: return dispatch_bc<GGML_F32, MODE>(p, B, cpl, grid, st);
    default: return hipErrorInvalidValue;
    }
}

int round_b(int b) { return b <= 1 ? 1 : (b <= 2 ? 2 : 4); }

GemvParams make_params(const DevMatrix &w, const float *x, int ldx, int b, int lpr_log2, int nchunks) {
    GemvParams p{};
    p.q = w.q;
    p.s = w.s;
    p.d = w.d;
    p.x = x;
    p.ldx = ldx;
    p.N = w.N;
    p.K = w.K;
    TypeInfo ti;
    type_info(w.type, &ti);
    p.nb = w.K / ti.block_elems;
    p.lpr_log2 = lpr_log2;
    p.nchunks = nchunks;
    p.b = b;
    p.mask_id = -1;
    return p;
}

int grid_for(const DevMatrix &w, int lpr_log2) {
    const int rpw = 64 >> lpr_log2;
    const int groups = (w.N + rpw - 1) / rpw;
    // each wave handles >= 2 row groups per iteration; cap the grid so that a wave
    // covers several groups of a large matrix (x is loaded once per wave)
    int waves = (groups + 1) / 2;
    int grid = (waves + 3) / 4;
    return grid < 1 ? 1 : (grid > 2048 ? 2048 : grid);
}

}  // namespace

int gemv_max_batch(const DevMatrix &w) {
    int l2, cpl, nc;
    if (!geometry(w, &l2, &cpl, &nc)) return 0;
    const int xw = xw_of(w.type);
    int best = 0;
    for (int b : {1, 2, 4})
        if (xw * b * cpl <= kMaxXRegs) best = b;
    return best;
}

hipError_t gemv(const DevMatrix &w, const float *x, int ldx, int b, float *y, int ldy, const float *bias, bool relu,
                hipStream_t st) {
    int l2, cpl, nc;
    if (b < 1 || b > gemv_max_batch(w) || !geometry(w, &l2, &cpl, &nc)) return hipErrorInvalidValue;
    GemvParams p = make_params(w, x, ldx, b, l2, nc);
    p.y = y;
    p.ldy = ldy;
    p.bias = bias;
    p.relu = relu ? 1 : 0;
    return dispatch<0>(w, p, round_b(b), cpl, grid_for(w, l2), st);
}

int gemv_argmax_parts(const DevMatrix &w, int b) {
    int l2, cpl, nc;
    if (!geometry(w, &l2, &cpl, &nc)) return 0;
    (void)b;
    return grid_for(w, l2);
}

hipError_t gemv_argmax(const DevMatrix &w, const float *x, int ldx, int b, int mask_id, float *pv, uint32_t *pi,
                       int *parts, hipStream_t st) {
    int l2, cpl, nc;
    if (b < 1 || b > gemv_max_batch(w) || !geometry(w, &l2, &cpl, &nc)) return hipErrorInvalidValue;
    GemvParams p = make_params(w, x, ldx, b, l2, nc);
    p.pv = pv;
    p.pi = pi;
    p.mask_id = mask_id;
    const int grid = grid_for(w, l2);
    *parts = grid;
    return dispatch<1>(w, p, round_b(b), cpl, grid, st);
}

}  // namespace mlg
