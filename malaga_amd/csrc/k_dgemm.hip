// Decode projections for batches of up to 64 rows (src/model.rs:552-612 at batch > 4):
// one launch per projection on the MFMA units, no split K, no reduction kernel.
//
// A workgroup owns one 16 x 16 output tile (grid N / 16 x M / 16).  Its NW waves split K:
// wave w takes the 256-wide K blocks w, w + NW, ..., so each X value is read by exactly
// one wave, straight from global memory into the A-operand registers (split there into
// f16 hi + lo), with no LDS staging.  The waves' partial tiles meet in LDS and are added
// in a fixed order; the epilogue then runs once per output, one output per thread of the
// first four waves.
//
// Loads complete in the order they are issued, and a wave that waits for one load waits
// for every load before it.  So each thread first requests what is needed first or is
// small (the LayerNorm operands, its epilogue operands), then the W quants of its first K
// block, then the X fragments in the order the slices use them; every load is
// unconditional (rows past M read row M - 1 and are never stored) and the wave index is a
// scalar, so that slice s waits for its own fragment and nothing later.
//
// Inputs are in fragment order (frag_index, device.hpp: whole cache lines per load),
// except PRO_RAW (row-major, the first layer's LayerNorm output).
//
// PRO_SPLIT: the input arrives split into f16 hi = f16(x) and lo = f16(x - hi), the form
// the A operand needs, written that way by its producer (the FFN-up projection, the
// attention), so no conversion is left here.
//
// PRO_LN: the input is LayerNorm(x) of the residual stream (fragment order, f32),
// normalized as the fragments arrive.  The row statistics are not recomputed: the launch that last wrote x
// (EPI_RESID) left the f64 sums of x and x^2 of every 16 columns beside it, and the
// prologue adds those P = K / 16 partials per row in a fixed order.
//
// Epilogues: EPI_STORE y = x W^T + bias (ReLU), f32 rows or split fragments; EPI_RESID x += x_in W^T + bias in place,
// plus the statistics of the new x; EPI_QKV q (f32) and K/V (f16, cache slot *step).
#include <type_traits>

#include "kernels.hpp"
#include "mfma_core.hpp"

namespace mlg {

namespace {

struct DArgs {
    WPtr w;
    const float *x;  // [M][ldx] input rows (PRO_LN: the residual stream; PRO_SPLIT: split rows)
    int ldx, M;
    const double *stats;  // PRO_LN: [M][P][2] sums of x and x^2 per 16 columns
    int P;
    const float *gamma, *beta;
    float eps;
    const float *bias;
    float *y;  // EPI_STORE [M][ldy] f32 rows, or split fragments (frag_out)
    int ldy, relu, frag_out;
    float *xres;        // EPI_RESID: the residual stream [M][N], fragment order
    double *stats_out;  // EPI_RESID: [M][N / 16][2]
    float *q;           // EPI_QKV: q [M][d], caches [M][H][slots][hd]
    __half *kc, *vc;
    float *kc32, *vc32;  // EPI_QKV with f32 caches (the generic path; kc / vc unused)
    int H, hd, slots;
    const uint32_t *step;
    const uint32_t *lens;  // k_dxattn: the rows' key counts (kc / vc: the cross caches [M][H][slots][hd])
};

enum DPro : int { PRO_RAW = 0, PRO_LN = 1, PRO_SPLIT = 2 };
enum DEpi : int { EPI_STORE = 0, EPI_RESID = 1, EPI_QKV = 2 };

constexpr int kDgMaxNW = 8;      // waves per workgroup at most (the K split)
constexpr int kDgMaxBPW = 4;     // K blocks per wave at most: K <= 8192
constexpr int kDgMaxLnK = 2048;  // LayerNorm projections: K = d_model <= 2048 (gamma, beta in LDS)
constexpr int kLnTPR = 16;                          // threads per row adding the statistics
constexpr int kLnQ = kDgMaxLnK / 16 / kLnTPR;       // partials per thread at most

// X fragment of one lane: XQ float4s of one (K block, slice)
template <int XQ>
struct DFrag {
    float4 x[XQ];
};

// Slice s of K block kb: acc[nt] += sc (W[nt] . X) over the slice's SK values (and - mn
// sum(X) for the k-quants with mins), for the W registers wrb[nt] of tile nt and the X
// fragment f of this lane (A row ln, k-group kq).  PRO_LN normalizes X with the row's mean
// mrow and 1 / std rrow and gamma | beta in gb (LDS, K each); PRO_SPLIT takes X already
// split into f16 hi | lo.  live false: the block is past the end and weighs 0.
template <int T, int NT, int PRO>
__device__ __forceinline__ void dg_slice(int kb, int s, int kq, const typename MW<T>::Regs (&wrb)[NT],
                                         const DFrag<MW<T>::SK / 16> &f, bool live, const float *gb, int K,
                                         float mrow, float rrow, f4_t (&acc)[NT]) {
    using W = MW<T>;
    constexpr int SK = W::SK, XQ = SK / 16;
    float sc[NT], mn[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        W::scale(wrb[nt], s, sc[nt], mn[nt]);
        sc[nt] = live ? sc[nt] : 0.f;
        mn[nt] = live ? mn[nt] : 0.f;
    }
    float v[SK / 4];
#pragma unroll
    for (int i = 0; i < (PRO == PRO_SPLIT ? 0 : XQ); ++i) {
        float4 e = f.x[i];
        if constexpr (PRO == PRO_LN) {
            const int k = kb * kStep + s * SK + kq * (SK / 4) + 4 * i;
            const float4 g = *reinterpret_cast<const float4 *>(gb + k), b = *reinterpret_cast<const float4 *>(gb + K + k);
            e = make_float4((e.x - mrow) * rrow * g.x + b.x, (e.y - mrow) * rrow * g.y + b.y,
                            (e.z - mrow) * rrow * g.z + b.z, (e.w - mrow) * rrow * g.w + b.w);
        }
        v[4 * i] = e.x;
        v[4 * i + 1] = e.y;
        v[4 * i + 2] = e.z;
        v[4 * i + 3] = e.w;
    }
    if constexpr (SK == 32) {
        h8_t ah, al;
        if constexpr (PRO == PRO_SPLIT) {
            // whole-vector shuffles (component access would keep the ring in memory)
            const h8_t p0 = __builtin_bit_cast(h8_t, f.x[0]), p1 = __builtin_bit_cast(h8_t, f.x[1]);
            ah = __builtin_shufflevector(p0, p1, 0, 1, 2, 3, 8, 9, 10, 11);
            al = __builtin_shufflevector(p0, p1, 4, 5, 6, 7, 12, 13, 14, 15);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                ah[i] = _Float16(v[i]);
                al[i] = _Float16(v[i] - float(ah[i]));
            }
        }
        f4_t xs = f4_t{0.f, 0.f, 0.f, 0.f};
        if constexpr (W::MIN) {  // per-row sums of the 32 X values: B = ones
            const h8_t ones = {_Float16(1), _Float16(1), _Float16(1), _Float16(1),
                               _Float16(1), _Float16(1), _Float16(1), _Float16(1)};
            xs = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, ones, xs, 0, 0, 0);
            xs = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, ones, xs, 0, 0, 0);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const h8_t bop = W::b(wrb[nt], s);
            f4_t tmp = f4_t{0.f, 0.f, 0.f, 0.f};
            tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bop, tmp, 0, 0, 0);
            tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bop, tmp, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[nt][r] = W::MIN ? fmaf(sc[nt], tmp[r], fmaf(-mn[nt], xs[r], acc[nt][r]))
                                    : fmaf(sc[nt], tmp[r], acc[nt][r]);
        }
    } else {
        h4_t ah, al;
        if constexpr (PRO == PRO_SPLIT) {
            const h8_t p0 = __builtin_bit_cast(h8_t, f.x[0]);
            ah = __builtin_shufflevector(p0, p0, 0, 1, 2, 3);
            al = __builtin_shufflevector(p0, p0, 4, 5, 6, 7);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ah[i] = _Float16(v[i]);
                al[i] = _Float16(v[i] - float(ah[i]));
            }
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const h4_t bop = W::b(wrb[nt], s);
            f4_t tmp = f4_t{0.f, 0.f, 0.f, 0.f};
            tmp = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bop, tmp, 0, 0, 0);
            tmp = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bop, tmp, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[nt][r] = fmaf(sc[nt], tmp[r], acc[nt][r]);
        }
    }
}

// The A operand (f16 hi | lo) of slice s of block kb for a 32-value slice: dg_slice's X
// arithmetic (PRO_LN: normalized with the row's statistics and gamma | beta; PRO_SPLIT:
// taken as it is).
template <int PRO>
__device__ __forceinline__ void dg_x32(int kb, int s, int kq, const DFrag<2> &f, const float *gb, int K, float mrow,
                                       float rrow, h8_t &ah, h8_t &al) {
    if constexpr (PRO == PRO_SPLIT) {
        const h8_t p0 = __builtin_bit_cast(h8_t, f.x[0]), p1 = __builtin_bit_cast(h8_t, f.x[1]);
        ah = __builtin_shufflevector(p0, p1, 0, 1, 2, 3, 8, 9, 10, 11);
        al = __builtin_shufflevector(p0, p1, 4, 5, 6, 7, 12, 13, 14, 15);
    } else {
        float v[8];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float4 e = f.x[i];
            if constexpr (PRO == PRO_LN) {
                const int k = kb * kStep + s * 32 + kq * 8 + 4 * i;
                const float4 g = *reinterpret_cast<const float4 *>(gb + k), b = *reinterpret_cast<const float4 *>(gb + K + k);
                e = make_float4((e.x - mrow) * rrow * g.x + b.x, (e.y - mrow) * rrow * g.y + b.y,
                                (e.z - mrow) * rrow * g.z + b.z, (e.w - mrow) * rrow * g.w + b.w);
            }
            v[4 * i] = e.x;
            v[4 * i + 1] = e.y;
            v[4 * i + 2] = e.z;
            v[4 * i + 3] = e.w;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ah[i] = _Float16(v[i]);
            al[i] = _Float16(v[i] - float(ah[i]));
        }
    }
}

// BPW: K blocks per wave (compile time, it sizes the fragment ring); NT: 16-column tiles
// per workgroup (1 or 2; with 2, each X fragment, once normalized and split, feeds two
// tiles); TL: W from the tile-major copy a.w.t (q6_K / q4_K); the wave count NW (4, 8, or
// up to NWL) is blockDim.x / 64.
template <int T, int BPW, int NT, int PRO, int EPI, bool TL, int NWL = kDgMaxNW>
__global__ __launch_bounds__(NWL * 64) void k_dgemm(DArgs a) {
    using W = MW<T>;
    constexpr int SK = W::SK, XQ = SK / 16;  // float4s of X per lane and slice
    constexpr int TN = 16 * NT, RS = TN + 1;  // columns of the tile; LDS row stride
    __shared__ float red[NWL * 16 * RS];
    __shared__ float lnm[16], lnr[16];
    __shared__ float gb[PRO == PRO_LN ? 2 * kDgMaxLnK : 1];  // PRO_LN: gamma | beta
    const int NW = int(blockDim.x) >> 6;
    const int t = threadIdx.x, lane = t & 63, ln = lane & 15, kq = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int K = a.w.K, nblk = K / kStep, n0 = blockIdx.x * TN, m0 = blockIdx.y * 16;
    // K block j of this wave; every wave runs BPW blocks, and a block past the end (K not
    // a multiple of NW x BPW blocks) is read at the last block and weighs 0
    auto blk = [&](int j) { return min(wv + j * NW, nblk - 1); };

    // PRO_LN operands: this thread's float4 of gamma and beta, and its share of the
    // statistics of row m0 + t / 16 (partials p = t % 16 + 16 q: a row's partials are
    // contiguous, so 16 lanes read 256 bytes)
    float4 gv = make_float4(0.f, 0.f, 0.f, 0.f), bv = gv;
    double2 sp[PRO == PRO_LN ? kLnQ : 1];
    if constexpr (PRO == PRO_LN) {
        const int gi = min(t, K / 4 - 1);
        gv = ld4(a.gamma, gi);
        bv = ld4(a.beta, gi);
        // waves 4..7 take no share: they read one address (no branch, which would make
        // the loads after it wait for these)
        const int m = wv < 4 ? min(m0 + (t >> 4), a.M - 1) : 0;
#pragma unroll
        for (int q = 0; q < kLnQ; ++q) {
            const int p = wv < 4 ? min((t & 15) + q * kLnTPR, a.P - 1) : 0;
            sp[q] = *reinterpret_cast<const double2 *>(a.stats + (size_t(m) * a.P + p) * 2);
        }
    }
    // epilogue operands of this thread's outputs o = t + 256 u: row m0 + o / TN, column
    // n0 + o % TN
    float bias_v[NT], xold[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) {
        const int o = t + 256 * u, omc = min(m0 + o / TN, a.M - 1), onc = min(n0 + o % TN, a.w.N - 1);
        bias_v[u] = a.bias ? a.bias[onc] : 0.f;
        xold[u] = 0.f;
        if constexpr (EPI == EPI_RESID) xold[u] = a.xres[frag_index(omc, onc & ~3, a.w.N) * 4 + (onc & 3)];
    }

    using WR = typename W::Regs;
    // W of the first K block, then the next block's when a block starts
    WR wr[2][NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) load_w<T, TL>(a.w, (n0 >> 4) + nt, ln, blk(0), kq, wr[0][nt]);

    // X fragment of (block kb, slice s): row m0 + ln, columns kb 256 + s SK + kq SK / 4
    // (fragment order: the tile's padding rows are stored)
    const float *xrow = a.x + size_t(min(m0 + ln, a.M - 1)) * a.ldx;
    const float4 *xfr = reinterpret_cast<const float4 *>(a.x);
    using Frag = DFrag<XQ>;
    auto load_x = [&](int kb, int s, Frag &f) {
        if constexpr (PRO != PRO_RAW) {
#pragma unroll
            for (int i = 0; i < XQ; ++i) f.x[i] = xfr[frag_index(m0 + ln, kb * kStep + s * SK + kq * (SK / 4) + 4 * i, K)];
        } else {
            const float4 *src = reinterpret_cast<const float4 *>(xrow + kb * kStep + s * SK + kq * (SK / 4));
#pragma unroll
            for (int i = 0; i < XQ; ++i) f.x[i] = src[i];
        }
    };
    // The (block, slice) items of this wave in order, D fragments in flight: item i uses
    // slot i % D, refilled with item i + D as soon as it is used.
    constexpr int NI = W::SLICES * BPW, D = NI < 16 / XQ ? NI : 16 / XQ;
    Frag buf[D];
#pragma unroll
    for (int i = 0; i < D; ++i) load_x(blk(i / W::SLICES), i % W::SLICES, buf[i]);
    // all of the above is requested before any of it is used
    __builtin_amdgcn_sched_barrier(0);

    float mrow = 0.f, rrow = 0.f;  // PRO_LN: mean and 1 / sqrt(var + eps) of this lane's row
    if constexpr (PRO == PRO_LN) {
        if (t < K / 4) {
            reinterpret_cast<float4 *>(gb)[t] = gv;
            reinterpret_cast<float4 *>(gb + K)[t] = bv;
        }
        if (wv < 4) {
            const int j = t & 15;
            double s1 = 0.0, s2 = 0.0;
#pragma unroll
            for (int q = 0; q < kLnQ; ++q)
                if (j + q * kLnTPR < a.P) {
                    s1 += sp[q].x;
                    s2 += sp[q].y;
                }
            s1 = group_sum_f64<kLnTPR>(s1);
            s2 = group_sum_f64<kLnTPR>(s2);
            if (j == 0) {
                const int ml = t >> 4;
                const double mu = s1 / K, var = fmax(s2 / K - mu * mu, 0.0);
                lnm[ml] = m0 + ml < a.M ? float(mu) : 0.f;
                lnr[ml] = m0 + ml < a.M ? float(1.0 / sqrt(var + double(a.eps))) : 0.f;
            }
        }
        __syncthreads();
        mrow = lnm[ln];
        rrow = lnr[ln];
    }

    f4_t acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    // slice s of block kb with the W registers wrb and the fragment f
    auto compute = [&](int kb, int s, const WR (&wrb)[NT], const Frag &f, bool live) {
        dg_slice<T, NT, PRO>(kb, s, kq, wrb, f, live, gb, K, mrow, rrow, acc);
    };
    static_for<0, BPW>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const int kb = blk(j);
        const bool live = wv + j * NW < nblk;  // scalar
        if constexpr (j + 1 < BPW)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
                load_w<T, TL>(a.w, (n0 >> 4) + nt, ln, blk(j + 1), kq, wr[(j + 1) & 1][nt]);
        if constexpr (W::FOLD) {
            // scales folded into B (mfma_core.hpp): the block's slices accumulate on the MFMA
            f4_t cb[NT], mb[NT];
            FoldPrep fp[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                cb[nt] = mb[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
                fp[nt] = fold_prep<W>(wr[j & 1][nt]);
            }
            static_for<0, W::SLICES>([&](auto sc) {
                constexpr int s = decltype(sc)::value, i = j * W::SLICES + s, r = i + D;
                h8_t ah, al;
                dg_x32<PRO>(kb, s, kq, buf[i % D], gb, K, mrow, rrow, ah, al);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) fold_slice<W>(wr[j & 1][nt], fp[nt], s, ah, al, cb[nt], mb[nt]);
                if constexpr (r < NI) {
                    __builtin_amdgcn_sched_barrier(0);
                    load_x(blk(r / W::SLICES), r % W::SLICES, buf[i % D]);
                }
            });
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) fold_flush<W>(wr[j & 1][nt], live, cb[nt], mb[nt], acc[nt]);
        } else {
            static_for<0, W::SLICES>([&](auto sc) {
                constexpr int s = decltype(sc)::value, i = j * W::SLICES + s, r = i + D;
                compute(kb, s, wr[j & 1], buf[i % D], live);
                if constexpr (r < NI) {
                    // the refill stays behind the compute that frees its slot (hoisted,
                    // it would hold a second set of fragments in registers)
                    __builtin_amdgcn_sched_barrier(0);
                    load_x(blk(r / W::SLICES), r % W::SLICES, buf[i % D]);
                }
            });
        }
    });

    // the waves' partial tiles (lane: column nt 16 + ln, rows 4 kq .. 4 kq + 3), added in
    // wave order
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wv * 16 + 4 * kq + r) * RS + nt * 16 + ln] = acc[nt][r];
    __syncthreads();
    if (wv >= 4) return;  // scalar: 256 NT outputs, NT per thread of the first four waves
    const uint32_t slot = EPI == EPI_QKV ? *a.step : 0u;
#pragma unroll
    for (int u = 0; u < NT; ++u) {
        const int o = t + 256 * u, ml = o / TN, c = o % TN, om = m0 + ml, on = n0 + c;
        const bool own = om < a.M && on < a.w.N;
        float v = red[ml * RS + c];
        for (int w = 1; w < NW; ++w) v += red[(w * 16 + ml) * RS + c];
        v += bias_v[u];
        if constexpr (EPI == EPI_STORE) {
            const float r = a.relu ? fmaxf(v, 0.f) : v;
            if (a.frag_out) {  // kernel argument: every lane takes this branch
                // lanes 4g .. 4g + 3 hold 4 consecutive columns of one row; the first
                // writes their [hi0..hi3 | lo0..lo3] fragment with one 16-byte store
                h4_t hv, lv;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float rj = __shfl(r, j, 4);
                    hv[j] = _Float16(rj);
                    lv[j] = _Float16(rj - float(hv[j]));
                }
                if (own && (c & 3) == 0) {
                    const uint2 hb = __builtin_bit_cast(uint2, hv), lb = __builtin_bit_cast(uint2, lv);
                    reinterpret_cast<uint4 *>(a.y)[frag_index(om, on, a.w.N)] = make_uint4(hb.x, hb.y, lb.x, lb.y);
                }
            } else if (own) {
                a.y[size_t(om) * a.ldy + on] = r;
            }
        } else if constexpr (EPI == EPI_QKV) {
            // K and V go to the f16 caches 8 columns (16 bytes) per store: lanes 8g .. 8g + 7
            // hold 8 consecutive columns of one row and one head (hd % 8 == 0)
            const int d = a.H * a.hd;
            h8_t hv;
#pragma unroll
            for (int j = 0; j < 8; ++j) hv[j] = _Float16(__shfl(v, j, 8));
            if (own) {
                const int cc = on < 2 * d ? on - d : on - 2 * d;
                const size_t off = ((size_t(om) * a.H + cc / a.hd) * a.slots + slot) * a.hd + cc % a.hd;
                if (on < d) {
                    a.q[size_t(om) * d + on] = v;
                } else if (a.kc32) {  // kernel argument: the same branch in every lane
                    (on < 2 * d ? a.kc32 : a.vc32)[off] = v;
                } else if ((c & 7) == 0) {
                    *reinterpret_cast<h8_t *>((on < 2 * d ? a.kc : a.vc) + off) = hv;
                }
            }
        } else {  // EPI_RESID: x += y, and the new x's sums per row and 16 columns (16 lanes)
            const float xn = own ? xold[u] + v : 0.f;
            if (own) a.xres[frag_index(om, on & ~3, a.w.N) * 4 + (on & 3)] = xn;
            const double s1 = group_sum_f64<16>(double(xn)), s2 = group_sum_f64<16>(double(xn) * double(xn));
            if (own && (c & 15) == 0) {
                double *sp_out = a.stats_out + (size_t(om) * (a.w.N >> 4) + (on >> 4)) * 2;
                sp_out[0] = s1;
                sp_out[1] = s2;
            }
        }
    }
}

// ---- decode projections with X resident in LDS (K <= 2048) ----
// The same products as k_dgemm for K = d_model, laid out the other way round: a workgroup
// of 8 waves owns one 16-row tile of X and stages it once, normalized (PRO_LN: k_dgemm's
// statistics order and expression) and split into f16 hi | lo, in LDS (128 KB at K =
// 2048).  Its NTW = 8 / KS column tiles of W go to the waves, KS waves per tile splitting
// the K blocks (wave kp takes blocks kp, kp + KS, ...), each wave streaming its W through
// a two-deep register ring with A fragments read from LDS.  So each X value is read from
// L2 and converted once per NTW column tiles (k_dgemm: once per 1, 2 or 4), and the first
// W jobs are requested before the staging, so that their HBM latency overlaps it.  The KS
// partial tiles of a column tile are added in K-part order through LDS; the sum then goes
// through the wave's LDS scratch to the row-major lane layout of the epilogues (4 columns
// of one row per lane: one 16-byte store per split fragment, float4 or f16 x 4 otherwise).
constexpr int kDrxWaves = 8;
constexpr int kDrxMaxDepth = 2;            // (tile, K block) jobs of W in flight per wave
constexpr int kDrxMaxKB = 8;               // K <= 2048
constexpr int kDrxScr = 16 * 17;           // a wave's 16 x 16 tile, row stride 17
__host__ __device__ constexpr int drx_xs(int K) { return K + 8; }  // halves per staged row

size_t drx_lds_bytes(int K, bool mins) {
    return size_t(16) * drx_xs(K) * 2 * sizeof(_Float16) + (mins ? size_t(K / 16) * 16 * sizeof(float) : 0) +
           size_t(kDrxWaves) * kDrxScr * sizeof(float) + 2 * 16 * sizeof(float);
}

template <int T, int KB, int KS, int PRO, int EPI, bool TL>
__global__ __launch_bounds__(kDrxWaves * 64) void k_drx(DArgs a) {
    using W = MW<T>;
    using WR = typename W::Regs;
    constexpr int SK = W::SK, NTW = kDrxWaves / KS, JPW = KB / KS;  // tiles per workgroup, jobs per wave
    constexpr int K = KB * kStep, XS = drx_xs(K);
    constexpr int NU = K / 128;  // staged 4-column units per thread (16 rows x K / 4 over 512 threads)
    static_assert(KB % KS == 0 && KB <= kDrxMaxKB, "K blocks split evenly over the waves of a tile");
    // two jobs of W in flight: every job requested at entry measured slower (config 5, 64
    // rows: 2.49 -> 2.57 ms per step, 214-254 VGPRs instead of 144-176)
    constexpr int kDrxDepth = JPW < kDrxMaxDepth ? JPW : kDrxMaxDepth;
    extern __shared__ __align__(16) unsigned char drx_lds[];
    _Float16 *xh = reinterpret_cast<_Float16 *>(drx_lds), *xl = xh + 16 * XS;
    constexpr bool XSUM = W::MIN && !W::FOLD;               // the min term from staged X sums
    float *xsum = reinterpret_cast<float *>(xl + 16 * XS);  // XSUM: [K / 16][16] sums of the staged X
    float *scr = xsum + (XSUM ? (K / 16) * 16 : 0);         // [waves][kDrxScr]
    float *lnm = scr + kDrxWaves * kDrxScr, *lnr = lnm + 16;
    const int t = threadIdx.x, lane = t & 63, ln = lane & 15, kq = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int m0 = blockIdx.y * 16, ntiles = (a.w.N + 15) / 16;
    const int tile = blockIdx.x * NTW + wv / KS, kp = wv % KS;
    const bool has_tile = tile < ntiles;  // scalar
    const int tl = min(tile, ntiles - 1), n0 = tl * 16;

    // 1. the first jobs' W (HBM), requested first
    WR ring[kDrxDepth];
#pragma unroll
    for (int u = 0; u < kDrxDepth; ++u) load_w<T, TL>(a.w, tl, ln, kp + min(u, JPW - 1) * KS, kq, ring[u]);
    __builtin_amdgcn_sched_barrier(0);

    // 2. epilogue operands of this lane's outputs: row m0 + er, columns n0 + 4 eq .. + 3
    const int er = lane >> 2, eq = lane & 3, em = min(m0 + er, a.M - 1), en = n0 + 4 * eq;
    float4 ebias = make_float4(0.f, 0.f, 0.f, 0.f), exold = ebias;
    uint32_t slot = 0;
    if (a.bias) ebias = ld4(a.bias, en >> 2);  // kernel argument: uniform
    if constexpr (EPI == EPI_RESID) exold = reinterpret_cast<const float4 *>(a.xres)[frag_index(em, en, a.w.N)];
    if constexpr (EPI == EPI_QKV) slot = *a.step;

    // 3. the X tile: unit i of this thread is row m0 + (t & 15), columns 4 cg .. 4 cg + 3 with
    // cg = t / 16 + 32 i (a wave reads 1 KB of whole lines per load).  PRO_LN: gamma and beta
    // pass through LDS (the start of the xh area, written only after they are read), so that
    // only X is held in registers across the load latency.
    const int xm = t & 15, xmc = min(m0 + xm, a.M - 1);
    const float4 *xfr = reinterpret_cast<const float4 *>(a.x);
    float4 xu[NU];
    double2 sp[KB];
    float4 gq = make_float4(0.f, 0.f, 0.f, 0.f), bq = gq;
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const int cg = (t >> 4) + 32 * i;
        if constexpr (PRO == PRO_RAW) xu[i] = ld4(a.x + size_t(xmc) * a.ldx, cg);
        else xu[i] = xfr[frag_index(xmc, 4 * cg, K)];
    }
    float *gbs = reinterpret_cast<float *>(xh);  // PRO_LN: gamma [K] | beta [K]
    if constexpr (PRO == PRO_LN) {
        if (t < K / 4) {  // scalar per wave (K / 4 is a multiple of 64)
            gq = ld4(a.gamma, t);
            bq = ld4(a.beta, t);
        }
        // statistics partials p = t % 16 + 16 q of row t / 16 (k_dgemm's order); waves 4..7
        // read row 0's and drop them
        const int m = wv < 4 ? min(m0 + (t >> 4), a.M - 1) : 0;
#pragma unroll
        for (int q = 0; q < KB; ++q)
            sp[q] = *reinterpret_cast<const double2 *>(a.stats + (size_t(m) * a.P + (t & 15) + q * kLnTPR) * 2);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PRO == PRO_LN) {
        if (t < K / 4) {
            reinterpret_cast<float4 *>(gbs)[t] = gq;
            reinterpret_cast<float4 *>(gbs + K)[t] = bq;
        }
        if (wv < 4) {
            double s1 = 0.0, s2 = 0.0;
#pragma unroll
            for (int q = 0; q < KB; ++q) {
                s1 += sp[q].x;
                s2 += sp[q].y;
            }
            s1 = group_sum_f64<kLnTPR>(s1);
            s2 = group_sum_f64<kLnTPR>(s2);
            if ((t & 15) == 0) {
                const int ml = t >> 4;
                const double mu = s1 / K, var = fmax(s2 / K - mu * mu, 0.0);
                lnm[ml] = m0 + ml < a.M ? float(mu) : 0.f;
                lnr[ml] = m0 + ml < a.M ? float(1.0 / sqrt(var + double(a.eps))) : 0.f;
            }
        }
        __syncthreads();
    }
    {
        const float mr = PRO == PRO_LN ? lnm[xm] : 0.f, rr = PRO == PRO_LN ? lnr[xm] : 0.f;
        uint4 hl[NU];  // [hi0..hi3 | lo0..lo3] of each unit
        float sums[NU];
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int cg = (t >> 4) + 32 * i;
            h4_t hv, lv;
            float sum = 0.f;
            if constexpr (PRO == PRO_SPLIT) {
                const uint4 u = __builtin_bit_cast(uint4, xu[i]);
                hv = __builtin_bit_cast(h4_t, make_uint2(u.x, u.y));
                lv = __builtin_bit_cast(h4_t, make_uint2(u.z, u.w));
#pragma unroll
                for (int j = 0; j < 4; ++j) sum += float(hv[j]) + float(lv[j]);
            } else {
                float v[4] = {xu[i].x, xu[i].y, xu[i].z, xu[i].w};
                if constexpr (PRO == PRO_LN) {
                    const float4 g = reinterpret_cast<const float4 *>(gbs)[cg], b = reinterpret_cast<const float4 *>(gbs + K)[cg];
                    v[0] = (v[0] - mr) * rr * g.x + b.x;
                    v[1] = (v[1] - mr) * rr * g.y + b.y;
                    v[2] = (v[2] - mr) * rr * g.z + b.z;
                    v[3] = (v[3] - mr) * rr * g.w + b.w;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    hv[j] = _Float16(v[j]);
                    lv[j] = _Float16(v[j] - float(hv[j]));
                }
                sum = (v[0] + v[1]) + (v[2] + v[3]);
            }
            const uint2 hb = __builtin_bit_cast(uint2, hv), lb = __builtin_bit_cast(uint2, lv);
            hl[i] = make_uint4(hb.x, hb.y, lb.x, lb.y);
            sums[i] = sum;
        }
        if constexpr (PRO == PRO_LN) __syncthreads();  // every read of gamma / beta is done
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int cg = (t >> 4) + 32 * i;
            *reinterpret_cast<uint2 *>(xh + xm * XS + 4 * cg) = make_uint2(hl[i].x, hl[i].y);
            *reinterpret_cast<uint2 *>(xl + xm * XS + 4 * cg) = make_uint2(hl[i].z, hl[i].w);
            if constexpr (XSUM) {
                // the 16 columns of chunk cg / 4 are in lanes xm, xm + 16, xm + 32, xm + 48
                float sum = sums[i];
                sum += __shfl_xor(sum, 16);
                sum += __shfl_xor(sum, 32);
                if (lane < 16) xsum[(cg >> 2) * 16 + xm] = sum;
            }
        }
    }
    __syncthreads();

    // 4. the jobs: K blocks kp + j KS of this wave's tile
    f4_t acc = f4_t{0.f, 0.f, 0.f, 0.f};
    auto job = [&](int kb, const WR &cur) {
        if constexpr (W::FOLD) {
            f4_t cb = f4_t{0.f, 0.f, 0.f, 0.f}, mb = cb;
            const FoldPrep fp = fold_prep<W>(cur);
#pragma unroll
            for (int s = 0; s < W::SLICES; ++s) {
                const int xo = ln * XS + kb * kStep + s * SK + kq * (SK / 4);
                const h8_t ah = *reinterpret_cast<const h8_t *>(xh + xo), al = *reinterpret_cast<const h8_t *>(xl + xo);
                fold_slice<W>(cur, fp, s, ah, al, cb, mb);
            }
            fold_flush<W>(cur, true, cb, mb, acc);
            return;
        }
#pragma unroll
        for (int s = 0; s < W::SLICES; ++s) {
            float sc, mn;
            W::scale(cur, s, sc, mn);
            const auto bop = W::b(cur, s);
            const int kx = kb * kStep + s * SK, xo = ln * XS + kx + kq * (SK / 4);
            f4_t tmp = f4_t{0.f, 0.f, 0.f, 0.f};
            if constexpr (SK == 32) {
                const h8_t ah = *reinterpret_cast<const h8_t *>(xh + xo), al = *reinterpret_cast<const h8_t *>(xl + xo);
                tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bop, tmp, 0, 0, 0);
                tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bop, tmp, 0, 0, 0);
            } else {
                const h4_t ah = *reinterpret_cast<const h4_t *>(xh + xo), al = *reinterpret_cast<const h4_t *>(xl + xo);
                tmp = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bop, tmp, 0, 0, 0);
                tmp = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bop, tmp, 0, 0, 0);
            }
            if constexpr (W::MIN) {
                const float *xsp = xsum + (kx >> 4) * 16 + 4 * kq;
                const float4 x0 = *reinterpret_cast<const float4 *>(xsp), x1 = *reinterpret_cast<const float4 *>(xsp + 16);
                const float xs[4] = {x0.x + x1.x, x0.y + x1.y, x0.z + x1.z, x0.w + x1.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] = fmaf(sc, tmp[r], fmaf(-mn, xs[r], acc[r]));
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] = fmaf(sc, tmp[r], acc[r]);
            }
        }
    };
    if (has_tile) {  // scalar
        static_for<0, JPW>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            job(kp + j * KS, ring[j % kDrxDepth]);
            if constexpr (j + kDrxDepth < JPW) {
                __builtin_amdgcn_sched_barrier(0);
                load_w<T, TL>(a.w, tl, ln, kp + (j + kDrxDepth) * KS, kq, ring[j % kDrxDepth]);
                __builtin_amdgcn_sched_barrier(0);
            }
        });
    }

    // 5. the tile's sum (K parts in order), moved to 4 columns of one row per lane
    float *my = scr + wv * kDrxScr;
    if constexpr (KS > 1) {
        *reinterpret_cast<f4_t *>(my + 4 * lane) = acc;
        __syncthreads();
        if (kp != 0 || !has_tile) return;  // scalar; no barrier below
#pragma unroll
        for (int k = 1; k < KS; ++k) {
            const f4_t o = *reinterpret_cast<const f4_t *>(scr + (wv + k) * kDrxScr + 4 * lane);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] += o[r];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's reads of its own slot are done
    } else {
        if (!has_tile) return;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) my[(4 * kq + r) * 17 + ln] = acc[r];
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    float v[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = my[er * 17 + 4 * eq + c];
    const int om = m0 + er;
    if (om >= a.M || en >= a.w.N) return;
    const float bv[4] = {ebias.x, ebias.y, ebias.z, ebias.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] += bv[c];

    // 6. epilogues
    if constexpr (EPI == EPI_STORE) {
        if (a.relu) {  // kernel argument
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = fmaxf(v[c], 0.f);
        }
        if (a.frag_out) {
            h4_t hv, lv;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                hv[c] = _Float16(v[c]);
                lv[c] = _Float16(v[c] - float(hv[c]));
            }
            const uint2 hb = __builtin_bit_cast(uint2, hv), lb = __builtin_bit_cast(uint2, lv);
            reinterpret_cast<uint4 *>(a.y)[frag_index(om, en, a.w.N)] = make_uint4(hb.x, hb.y, lb.x, lb.y);
        } else {
            *reinterpret_cast<float4 *>(a.y + size_t(om) * a.ldy + en) = make_float4(v[0], v[1], v[2], v[3]);
        }
    } else if constexpr (EPI == EPI_RESID) {
        const float xo[4] = {exold.x, exold.y, exold.z, exold.w};
        float xn[4];
        double s1 = 0.0, s2 = 0.0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            xn[c] = xo[c] + v[c];
            s1 += double(xn[c]);
            s2 += double(xn[c]) * double(xn[c]);
        }
        reinterpret_cast<float4 *>(a.xres)[frag_index(om, en, a.w.N)] = make_float4(xn[0], xn[1], xn[2], xn[3]);
        // the row's 16 columns are in lanes 4 er .. 4 er + 3
        s1 = group_sum_f64<4>(s1);
        s2 = group_sum_f64<4>(s2);
        if (eq == 0) {
            double *sp_out = a.stats_out + (size_t(om) * (a.w.N >> 4) + (en >> 4)) * 2;
            sp_out[0] = s1;
            sp_out[1] = s2;
        }
    } else {  // EPI_QKV: q f32; K / V into the caches at the step's slot (f16, or f32 with kc32)
        const int d = a.H * a.hd;
        if (en < d) {
            *reinterpret_cast<float4 *>(a.q + size_t(om) * d + en) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
            const int cc = en < 2 * d ? en - d : en - 2 * d;
            const size_t off = ((size_t(om) * a.H + cc / a.hd) * a.slots + slot) * a.hd + cc % a.hd;
            if (a.kc32) {  // kernel argument
                *reinterpret_cast<float4 *>((en < 2 * d ? a.kc32 : a.vc32) + off) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
                h4_t hv;
#pragma unroll
                for (int c = 0; c < 4; ++c) hv[c] = _Float16(v[c]);
                *reinterpret_cast<h4_t *>((en < 2 * d ? a.kc : a.vc) + off) = hv;
            }
        }
    }
}

// ---- the cross attention of a decode step in one launch ----
// crates/malaga-core/src/model.rs:573-578: q = cross_q(cross_norm(x)), then the cross
// attention of q over the source keys.  Workgroup (h, g), 8 waves, owns the RG = 8 / S
// rows [g RG, (g + 1) RG) and head h:
//   1. LN(x) of those rows, normalized once (k_dgemm's PRO_LN arithmetic: the statistics
//      partials added in the same order, the same expression) and split into f16 hi | lo
//      quads in LDS, [K / 4][RG];
//   2. q = LN(x) Wq^T + bq for the HD columns of the head on the MFMA units: wave w takes
//      the column tiles 2 (w % TG), + 1 of the head and K block w / TG (K <= 1024: one
//      block per wave), its A fragments from LDS (A-tile rows past RG repeat row RG - 1
//      and are dropped); the KG partial tiles are added in K-block order, then the bias:
//      k_dgemm's sums at its KG waves, so q is k_dgemm's bit for bit;
//   3. the attention of those rows and that head, S waves per (row, head) pair: wave
//      (pair p, split q) takes the keys SPL (S (c U + u) + q) + split of its lane splits
//      (k_attn_waves' loop, k_ops.hip: the same keys and order at the same S), with an online
//      softmax; at S > 1 the S partials meet in LDS and are rescaled to their common max.
// Every global operand is requested at the start: the W tiles, the X quads with gamma and
// beta, the first chunk of keys and values (it depends neither on q nor on the key count,
// so it arrives while the projection runs), then the statistics.  att goes out as split
// fragments (frag_index), the A operand of the cross out-projection.
constexpr int kDxHD = 64, kDxMaxBlocks = 256 / kDxHD, kDxMaxK = kDxMaxBlocks * kStep;

template <int T, int HD, int S, bool TL, typename KT>
__global__ __launch_bounds__(512) void k_dxattn(DArgs a) {
    using W = MW<T>;
    using WR = typename W::Regs;
    constexpr int SK = W::SK, XQ = SK / 16;
    constexpr int NT = 2, TG = HD / 32, KG = 8 / TG, RG = 8 / S;
    constexpr int TPK = HD / 8, SPL = 64 / TPK, U = 8 / S, RS = HD + 1, SLOT = HD + 2;
    constexpr int QN = kDxMaxK / 16 / kLnTPR;   // statistics partials per thread
    constexpr int SW = (16 * RG + 63) / 64;     // waves adding the statistics (16 lanes a row)
    __shared__ uint4 xs[kDxMaxK / 4 * RG];      // LN(x) quads [hi0..hi3 | lo0..lo3], [K / 4][RG]
    __shared__ float red[KG * RG * RS];
    __shared__ float qs[RG * HD];
    __shared__ float lnm[RG], lnr[RG];
    __shared__ float scr[8 * 512];                  // the waves' [64][8] attention sums
    __shared__ float slots[S > 1 ? 8 * SLOT : 1];   // S > 1: the waves' partials
    const int t = threadIdx.x, lane = t & 63, ln = lane & 15, kq = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int K = a.w.K, hh = blockIdx.x, m0 = blockIdx.y * RG;
    const int tile0 = hh * (HD / 16) + 2 * (wv % TG), kw = wv / TG;
    const int kb = min(kw, K / kStep - 1);
    const bool live = kw < K / kStep;  // scalar; a block past the end weighs 0

    WR wr[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) load_w<T, TL>(a.w, tile0 + nt, ln, kb, kq, wr[nt]);
    // quad f = t of the RG rows with its gamma and beta (threads t < K / 4: whole waves)
    const int f = min(t, K / 4 - 1);
    const float4 *xfr = reinterpret_cast<const float4 *>(a.x);
    float4 xv[RG], gv, bv;
    if (wv < K / 256) {  // scalar
#pragma unroll
        for (int r = 0; r < RG; ++r) xv[r] = xfr[frag_index(min(m0 + r, a.M - 1), 4 * f, K)];
        gv = ld4(a.gamma, f);
        bv = ld4(a.beta, f);
    }

    // this wave's (row, head) pair and the first chunk of its keys and values (keys past
    // the row's count are read at slot L - 1 and masked when used)
    const int pr = wv / S, ks = wv % S, bi = min(m0 + pr, a.M - 1);
    const int sub = lane % TPK, split = lane / TPK, L = a.slots, d = a.H * HD;
    const size_t kv0 = (size_t(bi) * a.H + hh) * size_t(L) * HD + sub * 8;
    // the caches in their precision: f16 (the graph step) or f32 (the generic decoder)
    const KT *kc, *vc;
    if constexpr (std::is_same_v<KT, float>) {
        kc = a.kc32;
        vc = a.vc32;
    } else {
        kc = a.kc;
        vc = a.vc;
    }
    Kv8<KT> kr[U], vr[U];
    auto key = [&](int c, int u) { return SPL * (S * (c * U + u) + ks) + split; };
    auto load_kv = [&](int c) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t o = kv0 + size_t(min(key(c, u), L - 1)) * HD;
            kr[u].load(kc + o);
            vr[u].load(vc + o);
        }
    };
    load_kv(0);
    const int n = int(a.lens[bi]);
    // all of the above is requested before any of it is used
    __builtin_amdgcn_sched_barrier(0);

    // the row statistics: partials p = t % 16 + 16 q of row t / 16 (rows past RG repeat
    // RG - 1), requested last by the waves that add them (a branch around loads whose
    // values outlive it would wait for them before the loads after it)
    if (wv < SW) {  // scalar
        const int j = t & 15, ml = t >> 4;
        const int m = min(m0 + min(ml, RG - 1), a.M - 1);
        double2 sp[QN];
#pragma unroll
        for (int q = 0; q < QN; ++q) {
            const int p = min(j + q * kLnTPR, a.P - 1);
            sp[q] = *reinterpret_cast<const double2 *>(a.stats + (size_t(m) * a.P + p) * 2);
        }
        double s1 = 0.0, s2 = 0.0;
#pragma unroll
        for (int q = 0; q < QN; ++q)
            if (j + q * kLnTPR < a.P) {
                s1 += sp[q].x;
                s2 += sp[q].y;
            }
        s1 = group_sum_f64<kLnTPR>(s1);
        s2 = group_sum_f64<kLnTPR>(s2);
        if (j == 0 && ml < RG) {
            const double mu = s1 / K, var = fmax(s2 / K - mu * mu, 0.0);
            lnm[ml] = m0 + ml < a.M ? float(mu) : 0.f;
            lnr[ml] = m0 + ml < a.M ? float(1.0 / sqrt(var + double(a.eps))) : 0.f;
        }
    }
    __syncthreads();
    if (wv < K / 256) {
#pragma unroll
        for (int r = 0; r < RG; ++r) {
            const float mr = lnm[r], rr = lnr[r];
            const float4 e = xv[r];
            const float v[4] = {(e.x - mr) * rr * gv.x + bv.x, (e.y - mr) * rr * gv.y + bv.y,
                                (e.z - mr) * rr * gv.z + bv.z, (e.w - mr) * rr * gv.w + bv.w};
            h4_t hv, lv;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                hv[j] = _Float16(v[j]);
                lv[j] = _Float16(v[j] - float(hv[j]));
            }
            const uint2 hb = __builtin_bit_cast(uint2, hv), lb = __builtin_bit_cast(uint2, lv);
            xs[f * RG + r] = make_uint4(hb.x, hb.y, lb.x, lb.y);
        }
    }
    __syncthreads();

    f4_t acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    const int ar = min(ln, RG - 1);
    // k_dgemm's arithmetic for the same slices (folded for q4_K / q5_K), so q equals its q
    f4_t cb[NT], mb[NT];
    FoldPrep fp[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        cb[nt] = mb[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
        if constexpr (W::FOLD) fp[nt] = fold_prep<W>(wr[nt]);
    }
    static_for<0, W::SLICES>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        DFrag<XQ> fr;
#pragma unroll
        for (int i = 0; i < XQ; ++i)
            fr.x[i] = __builtin_bit_cast(float4, xs[(kb * (kStep / 4) + s * (SK / 4) + kq * (SK / 16) + i) * RG + ar]);
        if constexpr (W::FOLD) {
            h8_t ah, al;
            dg_x32<PRO_SPLIT>(kb, s, kq, fr, nullptr, K, 0.f, 0.f, ah, al);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) fold_slice<W>(wr[nt], fp[nt], s, ah, al, cb[nt], mb[nt]);
        } else {
            dg_slice<T, NT, PRO_SPLIT>(kb, s, kq, wr, fr, live, nullptr, K, 0.f, 0.f, acc);
        }
    });
    if constexpr (W::FOLD)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) fold_flush<W>(wr[nt], live, cb[nt], mb[nt], acc[nt]);
    // the K blocks' partial tiles (lane: column nt 16 + ln, A rows 4 kq .. 4 kq + 3), then
    // q = their sum in K-block order + bias, in LDS
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (4 * kq + r < RG) red[(kw * RG + 4 * kq + r) * RS + (wv % TG) * 32 + nt * 16 + ln] = acc[nt][r];
    __syncthreads();
    for (int o = t; o < RG * HD; o += 512) {
        const int r = o / HD, c = o % HD;
        float v = red[r * RS + c];
        for (int w = 1; w < KG; ++w) v += red[(w * RG + r) * RS + c];
        v += a.bias ? a.bias[hh * HD + c] : 0.f;
        qs[o] = v;
    }
    __syncthreads();

    const float *qp = qs + pr * HD + sub * 8;
    const float4 qa = *reinterpret_cast<const float4 *>(qp), qb = *reinterpret_cast<const float4 *>(qp + 4);
    float m = -INFINITY, l = 0.f;
    float o8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int c = 0; SPL * (S * c * U + ks) < n; ++c) {  // wave-uniform; chunk 0 is in flight
        if (c) load_kv(c);
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
        for (int e = 0; e < 8; ++e) o8[e] *= rs;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool in = key(c, u) < n;
            const float pj = in ? expf(sc[u] - mnew) : 0.f;
            l += pj;
            float vv[8];
            vr[u].unpack(vv, in);
#pragma unroll
            for (int e = 0; e < 8; ++e) o8[e] = fmaf(pj, vv[e], o8[e]);
        }
        m = mnew;
    }
    // every lane of a split holds that split's sum: count each split once
    const float lsum = wave_sum(sub == 0 ? l : 0.f);
    float *wsc = scr + wv * 512;
#pragma unroll
    for (int e = 0; e < 8; ++e) wsc[lane * 8 + e] = o8[e];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    // split fragments [hi0..hi3 | lo0..lo3] of att[bi][h HD + 4 e4 ..], one lane per 4 values
    auto store4 = [&](int e4, const float (&v)[4]) {
        h4_t hv, lv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hv[j] = _Float16(v[j]);
            lv[j] = _Float16(v[j] - float(hv[j]));
        }
        const uint2 hb = __builtin_bit_cast(uint2, hv), lb = __builtin_bit_cast(uint2, lv);
        reinterpret_cast<uint4 *>(a.y)[frag_index(bi, hh * HD + 4 * e4, d)] = make_uint4(hb.x, hb.y, lb.x, lb.y);
    };
    const bool own = m0 + pr < a.M;  // scalar
    if constexpr (S == 1) {
        const float inv = 1.f / lsum;
        if (own)
            for (int e4 = lane; e4 < HD / 4; e4 += 64) {
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int e = 4 * e4 + j;
                    float o = 0.f;
#pragma unroll
                    for (int s2 = 0; s2 < SPL; ++s2) o += wsc[(s2 * TPK + e / 8) * 8 + e % 8];
                    v[j] = o * inv;
                }
                store4(e4, v);
            }
    } else {
        // this wave's partial: sum_j p_j v_j over its keys, its max (-inf without keys) and sum p_j
        float *slot = slots + wv * SLOT;
        for (int e = lane; e < HD; e += 64) {
            float o = 0.f;
#pragma unroll
            for (int s2 = 0; s2 < SPL; ++s2) o += wsc[(s2 * TPK + e / 8) * 8 + e % 8];
            slot[e] = o;
        }
        if (lane == 0) {
            slot[HD] = m;
            slot[HD + 1] = lsum;
        }
        __syncthreads();
        if (ks == 0 && own) {  // scalar; the pair's wave 0 has key 0, so its max is finite
            const float *ps = slots + wv * SLOT;
            float mx = ps[HD];
#pragma unroll
            for (int q = 1; q < S; ++q) mx = fmaxf(mx, ps[q * SLOT + HD]);
            float ew[S], den = 0.f;
#pragma unroll
            for (int q = 0; q < S; ++q) {
                ew[q] = expf(ps[q * SLOT + HD] - mx);
                den += ew[q] * ps[q * SLOT + HD + 1];
            }
            const float inv = 1.f / den;
            for (int e4 = lane; e4 < HD / 4; e4 += 64) {
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float o = 0.f;
#pragma unroll
                    for (int q = 0; q < S; ++q) o += ew[q] * ps[q * SLOT + 4 * e4 + j];
                    v[j] = o * inv;
                }
                store4(e4, v);
            }
        }
    }
}


// Waves of S per (row, head) pair: 4 (2 rows per workgroup)
constexpr int kDxSplit = 4;
inline int dx_rows() { return 8 / kDxSplit; }
// Heads of 64 and K <= 1024 (d_model of the 600M and 1.3B checkpoints): one K block per
// wave; other shapes keep the two launches.

template <int T, typename KT>
hipError_t launch_dxattn_k(const DArgs &a, hipStream_t st) {
    const dim3 grid(unsigned(a.H), unsigned((a.M + dx_rows() - 1) / dx_rows()));
    if constexpr (T == GGML_Q6_K || T == GGML_Q4_K) {
        if (a.w.t) {
            hipLaunchKernelGGL((k_dxattn<T, kDxHD, kDxSplit, true, KT>), grid, dim3(512), 0, st, a);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((k_dxattn<T, kDxHD, kDxSplit, false, KT>), grid, dim3(512), 0, st, a);
    return hipGetLastError();
}

template <int T>
hipError_t launch_dxattn_t(const DArgs &a, hipStream_t st) {
    return a.kc32 ? launch_dxattn_k<T, float>(a, st) : launch_dxattn_k<T, __half>(a, st);
}

// The K split: 4 waves up to four K blocks (K <= 1024), else 8 waves of 1, 2 or 4 blocks.
inline int dg_waves(int nblk) { return nblk <= 4 ? 4 : kDgMaxNW; }
inline int dg_bpw(int nblk) {
    const int nw = dg_waves(nblk), per = (nblk + nw - 1) / nw;
    return per <= 1 ? 1 : per <= 2 ? 2 : 4;
}

// Two column tiles per workgroup where one tile each would take 1.5 workgroups per CU or
// more: the normalized, split X then feeds both (at 32 rows: QKV 7.7 us instead of 9.3,
// FFN-up 7.4 instead of 9.3).  Four where one each would take six per CU (the 3.3B
// model's QKV and FFN-up at 64 rows): every workgroup reads its 16 rows of X once for
// 64 columns.
constexpr int kDgWideGrid = 384;
constexpr int kDgWiderGrid = 1536;

template <int T, int BPW, int PRO, int EPI, bool TL>
hipError_t launch_dgemm_l(const DArgs &a, hipStream_t st) {
    const unsigned gy = unsigned((a.M + 15) / 16), block = unsigned(dg_waves(a.w.K / kStep) * 64);
    const unsigned tiles1 = unsigned((a.w.N + 15) / 16);
    if constexpr (EPI != EPI_RESID && BPW == 1) {
        if (tiles1 * gy >= unsigned(kDgWiderGrid)) {
            hipLaunchKernelGGL((k_dgemm<T, BPW, 4, PRO, EPI, TL>), dim3((a.w.N + 63) / 64, gy), dim3(block), 0, st, a);
            return hipGetLastError();
        }
    }
    if (tiles1 * gy >= unsigned(kDgWideGrid)) {
        hipLaunchKernelGGL((k_dgemm<T, BPW, 2, PRO, EPI, TL>), dim3((a.w.N + 31) / 32, gy), dim3(block), 0, st, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((k_dgemm<T, BPW, 1, PRO, EPI, TL>), dim3(tiles1, gy), dim3(block), 0, st, a);
    return hipGetLastError();
}

// q6_K / q4_K with its tile-major copy reads that copy
template <int T, int BPW, int PRO, int EPI>
hipError_t launch_dgemm(const DArgs &a, hipStream_t st) {
    if constexpr (T == GGML_Q6_K || T == GGML_Q4_K) {
        if (a.w.t) return launch_dgemm_l<T, BPW, PRO, EPI, true>(a, st);
    }
    return launch_dgemm_l<T, BPW, PRO, EPI, false>(a, st);
}

// A residual projection of 9..16 K blocks (ffn_down at FFN width 4096): 16 waves of one
// block each (1024 threads; the one-block variants fit the 128 VGPRs that allows) rather
// than 8 waves of two
constexpr int kDgWaves16 = 16;
template <int T, int PRO, int EPI>
hipError_t launch_dgemm16(const DArgs &a, hipStream_t st) {
    const dim3 grid(unsigned((a.w.N + 15) / 16), unsigned((a.M + 15) / 16)), block(kDgWaves16 * 64);
    if constexpr (T == GGML_Q6_K || T == GGML_Q4_K) {
        if (a.w.t) {
            hipLaunchKernelGGL((k_dgemm<T, 1, 1, PRO, EPI, true, kDgWaves16>), grid, block, 0, st, a);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((k_dgemm<T, 1, 1, PRO, EPI, false, kDgWaves16>), grid, block, 0, st, a);
    return hipGetLastError();
}

// only the residual projections (ffn_down: K = the FFN width) take more than one K
// block per wave
template <int T, int PRO, int EPI>
hipError_t launch_dgemm_m(const DArgs &a, hipStream_t st) {
    const int bpw = dg_bpw(a.w.K / kStep);
    if constexpr (EPI == EPI_RESID && PRO == PRO_SPLIT) {
        if (a.w.K / kStep > kDgMaxNW && a.w.K / kStep <= kDgWaves16) return launch_dgemm16<T, PRO, EPI>(a, st);
    }
    if constexpr (EPI == EPI_RESID) {
        if (bpw == 4) return launch_dgemm<T, 4, PRO, EPI>(a, st);
        if (bpw == 2) return launch_dgemm<T, 2, PRO, EPI>(a, st);
    } else if (bpw != 1) {
        return hipErrorInvalidValue;  // K > 2048 in a LayerNorm / QKV projection: not a decoder shape
    }
    return launch_dgemm<T, 1, PRO, EPI>(a, st);
}

// Resident-X launches (k_drx): q4_K / q6_K with their tile-major copies, K = 2048 (the 3.3B
// model's d_model), N a multiple of 16, and enough column tiles for 128 workgroups of 8
// tiles (QKV and FFN-up at 64 rows).  Measured against k_dgemm (rocprofv3, same box):
// at K = 2048 and 64 rows QKV 24.1 -> 16.9 us and FFN-up 24.3 -> 17.4 us, but the d-wide
// projections (N = 2048, two waves per tile) 6.7 -> 11.0 us and 9.4 -> 12.7 us; at K = 1024
// and 32 rows no projection gained (FFN-up 7.4 -> 8.6 us): staging 16 rows of X costs
// more than it saves when a workgroup feeds it to few columns.
constexpr int kDrxMinGrid = 128;

bool drx_ok(const DevMatrix &w, int M) {
    const int gx = (w.N / 16 + kDrxWaves - 1) / kDrxWaves, gy = (M + 15) / 16;
    return (w.type == GGML_Q4_K || w.type == GGML_Q6_K) && w.tm && w.K == 2048 && w.N % 16 == 0 && M >= 1 &&
           M <= kDgemmMaxRows && gx * gy >= kDrxMinGrid;
}

template <int T, int KB, int KS, int PRO, int EPI>
hipError_t launch_drx_k(const DArgs &a, hipStream_t st) {
    const size_t lds = drx_lds_bytes(KB * kStep, MW<T>::MIN && !MW<T>::FOLD);
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_drx<T, KB, KS, PRO, EPI, true>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (attr != hipSuccess) return attr;
    constexpr int ntw = kDrxWaves / KS;
    const dim3 grid(unsigned((a.w.N / 16 + ntw - 1) / ntw), unsigned((a.M + 15) / 16));
    hipLaunchKernelGGL((k_drx<T, KB, KS, PRO, EPI, true>), grid, dim3(kDrxWaves * 64), lds, st, a);
    return hipGetLastError();
}

template <int PRO, int EPI>
hipError_t launch_drx(const DevMatrix &w, const DArgs &a, hipStream_t st) {
    if (w.type == GGML_Q4_K) return launch_drx_k<GGML_Q4_K, 8, 1, PRO, EPI>(a, st);
    return launch_drx_k<GGML_Q6_K, 8, 1, PRO, EPI>(a, st);
}

template <int PRO, int EPI>
hipError_t launch_dgemm_t(const DevMatrix &w, const DArgs &a, hipStream_t st) {
    switch (w.type) {
    case GGML_Q4_K: return launch_dgemm_m<GGML_Q4_K, PRO, EPI>(a, st);
    case GGML_Q5_K: return launch_dgemm_m<GGML_Q5_K, PRO, EPI>(a, st);
    case GGML_Q6_K: return launch_dgemm_m<GGML_Q6_K, PRO, EPI>(a, st);
    case GGML_Q8_0: return launch_dgemm_m<GGML_Q8_0, PRO, EPI>(a, st);
    case GGML_F16: return launch_dgemm_m<GGML_F16, PRO, EPI>(a, st);
    default: return hipErrorInvalidValue;
    }
}

DArgs dargs(const DevMatrix &w, const float *x, int ldx, int M, const DgemmLn *ln, const float *bias) {
    DArgs a{};
    a.w = wptr_of(w);
    a.x = x;
    a.ldx = ldx;
    a.M = M;
    a.bias = bias;
    if (ln) {
        a.stats = ln->stats;
        a.P = w.K / 16;
        a.gamma = ln->g;
        a.beta = ln->b;
        a.eps = ln->eps;
    }
    return a;
}

bool dgemm_args_ok(const DevMatrix &w, const float *x, int ldx, int M, const DgemmLn *ln) {
    // ldx % 8: rows of the split planes start on 16 bytes too
    return dgemm_supported(w, M) && x && ldx % 8 == 0 && ldx >= w.K && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
           (!ln || (ln->stats && ln->g && ln->b && reinterpret_cast<uintptr_t>(ln->g) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(ln->b) % 16 == 0));
}

}  // namespace

bool dgemm_supported(const DevMatrix &w, int M) {
    return gemm_mfma_supported(w) && M >= 1 && M <= kDgemmMaxRows && w.K / kStep <= kDgMaxBPW * kDgMaxNW;
}

hipError_t dgemm_store(const DevMatrix &w, const float *x, int ldx, int M, const DgemmLn *ln, const float *bias,
                       bool relu, float *y, int ldy, hipStream_t st, bool y_split, bool resident) {
    if (!dgemm_args_ok(w, x, ldx, M, ln) || !y || ldy < w.N) return hipErrorInvalidValue;
    // split fragments: 16-byte aligned, whole slices of 16 columns
    if (y_split && (w.N % 16 || reinterpret_cast<uintptr_t>(y) % 16)) return hipErrorInvalidValue;
    DArgs a = dargs(w, x, ldx, M, ln, bias);
    a.y = y;
    a.frag_out = y_split ? 1 : 0;
    a.ldy = ldy;
    a.relu = relu ? 1 : 0;
    // row-major stores of 4 columns need 16-byte rows
    if (resident && ln && drx_ok(w, M) && (y_split || (ldy % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0)))
        return launch_drx<PRO_LN, EPI_STORE>(w, a, st);
    return ln ? launch_dgemm_t<PRO_LN, EPI_STORE>(w, a, st) : launch_dgemm_t<PRO_RAW, EPI_STORE>(w, a, st);
}

hipError_t dgemm_resid(const DevMatrix &w, const float *x, int ldx, int M, const float *bias, float *xres,
                       double *stats_out, hipStream_t st, bool x_split) {
    if (!dgemm_args_ok(w, x, ldx, M, nullptr) || !xres || !stats_out || w.N % 16) return hipErrorInvalidValue;
    DArgs a = dargs(w, x, ldx, M, nullptr, bias);
    a.xres = xres;
    a.stats_out = stats_out;
    if (x_split && drx_ok(w, M)) return launch_drx<PRO_SPLIT, EPI_RESID>(w, a, st);
    if (x_split) return launch_dgemm_t<PRO_SPLIT, EPI_RESID>(w, a, st);
    return launch_dgemm_t<PRO_RAW, EPI_RESID>(w, a, st);
}

namespace {
hipError_t dgemm_qkv_any(const DevMatrix &w, const float *x, int ldx, int M, const DgemmLn *ln, const float *bias,
                         int H, int hd, int slots, const uint32_t *step, float *q, __half *kc, __half *vc, float *kc32,
                         float *vc32, hipStream_t st) {
    const void *k = kc ? static_cast<const void *>(kc) : kc32, *v = vc ? static_cast<const void *>(vc) : vc32;
    if (!dgemm_args_ok(w, x, ldx, M, ln) || w.N != 3 * H * hd || hd % 8 || !q || !k || !v || !step ||
        reinterpret_cast<uintptr_t>(k) % 16 || reinterpret_cast<uintptr_t>(v) % 16)
        return hipErrorInvalidValue;
    DArgs a = dargs(w, x, ldx, M, ln, bias);
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.kc32 = kc32;
    a.vc32 = vc32;
    a.H = H;
    a.hd = hd;
    a.slots = slots;
    a.step = step;
    // the resident-X kernel stores 4 columns per lane: heads of 4 k, rows of 16 bytes
    if (drx_ok(w, M) && hd % 4 == 0 && (ln || (ldx % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0)))
        return ln ? launch_drx<PRO_LN, EPI_QKV>(w, a, st) : launch_drx<PRO_RAW, EPI_QKV>(w, a, st);
    return ln ? launch_dgemm_t<PRO_LN, EPI_QKV>(w, a, st) : launch_dgemm_t<PRO_RAW, EPI_QKV>(w, a, st);
}
}  // namespace

hipError_t dgemm_qkv(const DevMatrix &w, const float *x, int ldx, int M, const DgemmLn *ln, const float *bias, int H,
                     int hd, int slots, const uint32_t *step, float *q, __half *kc, __half *vc, hipStream_t st) {
    return dgemm_qkv_any(w, x, ldx, M, ln, bias, H, hd, slots, step, q, kc, vc, nullptr, nullptr, st);
}

hipError_t dgemm_qkv(const DevMatrix &w, const float *x, int ldx, int M, const DgemmLn *ln, const float *bias, int H,
                     int hd, int slots, const uint32_t *step, float *q, float *kc, float *vc, hipStream_t st) {
    return dgemm_qkv_any(w, x, ldx, M, ln, bias, H, hd, slots, step, q, nullptr, nullptr, kc, vc, st);
}

bool dgemm_cross_attn_supported(const DevMatrix &w, int M, int H, int hd) {
    return dgemm_supported(w, M) && hd == kDxHD && H >= 1 && w.N == H * hd && w.K / kStep <= kDxMaxBlocks;
}

namespace {
hipError_t dgemm_cross_attn_any(const DevMatrix &w, const float *x, int M, const DgemmLn &ln, const float *bias,
                                const __half *K, const __half *V, const float *K32, const float *V32, int H, int hd,
                                int L, const uint32_t *lens, float *att, hipStream_t st) {
    const void *k = K ? static_cast<const void *>(K) : K32, *v = V ? static_cast<const void *>(V) : V32;
    if (!dgemm_cross_attn_supported(w, M, H, hd) || !dgemm_args_ok(w, x, w.K, M, &ln) || !k || !v || !lens || !att ||
        L < 1 || reinterpret_cast<uintptr_t>(k) % 16 || reinterpret_cast<uintptr_t>(v) % 16 ||
        reinterpret_cast<uintptr_t>(att) % 16)
        return hipErrorInvalidValue;
    DArgs a = dargs(w, x, w.K, M, &ln, bias);
    a.kc = const_cast<__half *>(K);
    a.vc = const_cast<__half *>(V);
    a.kc32 = const_cast<float *>(K32);
    a.vc32 = const_cast<float *>(V32);
    a.H = H;
    a.hd = hd;
    a.slots = L;
    a.lens = lens;
    a.y = att;
    switch (w.type) {
    case GGML_Q4_K: return launch_dxattn_t<GGML_Q4_K>(a, st);
    case GGML_Q5_K: return launch_dxattn_t<GGML_Q5_K>(a, st);
    case GGML_Q6_K: return launch_dxattn_t<GGML_Q6_K>(a, st);
    case GGML_Q8_0: return launch_dxattn_t<GGML_Q8_0>(a, st);
    case GGML_F16: return launch_dxattn_t<GGML_F16>(a, st);
    default: return hipErrorInvalidValue;
    }
}
}  // namespace

hipError_t dgemm_cross_attn(const DevMatrix &w, const float *x, int M, const DgemmLn &ln, const float *bias,
                            const __half *K, const __half *V, int H, int hd, int L, const uint32_t *lens, float *att,
                            hipStream_t st) {
    return dgemm_cross_attn_any(w, x, M, ln, bias, K, V, nullptr, nullptr, H, hd, L, lens, att, st);
}

hipError_t dgemm_cross_attn(const DevMatrix &w, const float *x, int M, const DgemmLn &ln, const float *bias,
                            const float *K, const float *V, int H, int hd, int L, const uint32_t *lens, float *att,
                            hipStream_t st) {
    return dgemm_cross_attn_any(w, x, M, ln, bias, nullptr, nullptr, K, V, H, hd, L, lens, att, st);
}

}  // namespace mlg
