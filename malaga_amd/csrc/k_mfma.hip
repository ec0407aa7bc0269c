// Dequant GEMM on the MFMA units (src/model.rs:463-477 encoder prefill, and the
// projections of decode batches too large for the register GEMV):
//   Y[m][n] = sum_k X[m][k] W[n][k] + bias[n] (+ R[m][n]) (relu)
//
// Exactness: the integer quants (q4_K / q5_K nibbles, q6_K 6-bit values - 32,
// q8_0 int8) are exact in f16, so the MFMA multiplies them by X, which is split
// into two f16 terms x = hi + lo (|x - hi - lo| <= 2^-22 |x|), with f32
// accumulation; block scales and k-quant mins are applied per sub-block in f32:
//   sum_k w_k x_k = d sc * sum_k q_k x_k - dmin m * sum_k x_k,
// except for q6_K, whose int8 group scales are folded into B as the exact pair
// bh + bl = q sc (MW<q6_K>::b_split): a super-block's 8 slices of 32 chain in the
// 16x16x32 MFMA's C operand and d is applied once per block.
//
// Tiling: a workgroup (4 waves) owns 64 rows of W (16 per wave) and BM rows of X.
// K is consumed in steps of 256 (one k-quant super-block): the X step is staged
// in LDS as hi/lo f16 plus per-16 sums, while the next step's X and W are in
// flight in registers.  Each wave keeps its W rows in registers in the MFMA
// B-operand layout (lane l: row l % 16, k-group l / 16) and reads A (X) from LDS.
// f16 MFMA operand conversion of quant bytes uses v_perm (byte -> 0x64xx = 1024 +
// byte) and one packed f16 subtraction.
#include "kernels.hpp"
#include "mfma_core.hpp"

#include <algorithm>

namespace mlg {

namespace {

// LDS row stride of the staged X (halves).  272 (136 dwords): the A-fragment reads and the
// 16-byte staging stores have no bank conflicts (rocprofv3: 264 and 280 left 49-65 K conflict
// cycles per CU in each encoder GEMM launch, 272 none for q6_K).  The resident-X LM head
// (k_mfma_rx) uses the same 8-mod-64-dword stride (rx_stride); k_drx keeps K + 8 (its bank
// conflicts are off the critical path)
constexpr int kXS = kStep + 16;

constexpr int kTileN = 64;        // W rows per workgroup

// X staging of one 256-wide K step into LDS as f16 hi / lo (+ per-16 sums for the
// formats with mins).  Each thread converts chunks of 8 values and writes them as one
// 16-byte store; 16 consecutive lanes take 16 consecutive chunks of one row, so each
// store of 16 lanes covers 256 contiguous bytes of LDS (no bank conflicts).  Thread t:
// rows t / 16 + (NTH / 16) u, chunks t % 16 + 16 h (32 chunks per row and step).
// Chunk c holds x[8 c .. 8 c + 7], or for split-B types the two 4-value groups that
// split_pos puts there: x[32 (c / 4) + 4 (c % 4) + e] and x[32 (c / 4) + 16 + 4 (c % 4) + e].
template <int BM, int NTH, bool SPLIT>
struct XStage {
    static constexpr int R = NTH / 16, RP = BM / R;  // rows per pass, row passes
    static_assert(RP >= 1 && BM % R == 0, "X tile / thread count");
    float4 v[RP][2][2];  // [row pass][chunk h][half]
    const float *src[RP];
    bool ok[RP];
    int cl, rg;
    __device__ void init(const float *x, int ldx, int m0, int M, int t) {
        cl = t & 15, rg = t >> 4;
#pragma unroll
        for (int u = 0; u < RP; ++u) {
            const int m = m0 + rg + R * u;
            ok[u] = m < M;
            src[u] = x + size_t(ok[u] ? m : 0) * ldx;
        }
    }
    __device__ static int koff(int c, int half) {
        if constexpr (SPLIT) return 32 * (c >> 2) + 16 * half + 4 * (c & 3);
        else return 8 * c + 4 * half;
    }
    __device__ void load(int kb) {
#pragma unroll
        for (int u = 0; u < RP; ++u)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int f = 0; f < 2; ++f)
                    v[u][h][f] = ok[u] ? *reinterpret_cast<const float4 *>(src[u] + size_t(kb) * kStep +
                                                                         koff(cl + 16 * h, f))
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    template <bool SUMS>
    __device__ void store(_Float16 *xh, _Float16 *xl, float *xsum) const {
#pragma unroll
        for (int u = 0; u < RP; ++u)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int m = rg + R * u, c = cl + 16 * h;
                const float e[8] = {v[u][h][0].x, v[u][h][0].y, v[u][h][0].z, v[u][h][0].w,
                                    v[u][h][1].x, v[u][h][1].y, v[u][h][1].z, v[u][h][1].w};
                h8_t hv, lv;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    hv[i] = _Float16(e[i]);
                    lv[i] = _Float16(e[i] - float(hv[i]));
                }
                *reinterpret_cast<h8_t *>(xh + m * kXS + 8 * c) = hv;
                *reinterpret_cast<h8_t *>(xl + m * kXS + 8 * c) = lv;
                if constexpr (SUMS) {  // 16-value sums: this chunk and the next (lane cl ^ 1)
                    float sm = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
                    sm += dpp_mov<kDppXor1>(sm);
                    if (!(cl & 1)) xsum[(c >> 1) * BM + m] = sm;
                }
            }
    }
};

struct MfmaArgs {
    WPtr w;
    const float *x;
    int ldx, M;
    float *y;
    int ldy;
    const float *bias, *R;
    int ldr, relu;
    float *part;  // split K: raw sums [gridDim.z][M][N], epilogue in k_splitk_reduce
    int mask_id;  // k_mfma_w MODE 1: row index never selected (-1: none)
    float *pv;    // k_mfma_w MODE 1: argmax partials [M][parts], one per workgroup
    uint32_t *pi;
    int parts;
};


// TL (all three GEMM kernels): W from the tile-major copy a.w.t (q6_K / q4_K)
template <int T, int BM, bool TL>
__global__ __launch_bounds__(256) void k_mfma(MfmaArgs a) {
    using W = MW<T>;
    constexpr int MT = BM / 16;     // 16-row tiles of X
    __shared__ _Float16 xh[BM * kXS], xl[BM * kXS];
    __shared__ float xsum[16 * BM];  // [16-slice][m]
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int kq = lane >> 4, ln = lane & 15;
    const int n0 = blockIdx.x * kTileN + 16 * w;
    const int m0 = blockIdx.y * BM;
    // K steps [kb0, kb1) of this split
    const int nsteps = a.w.K / kStep, ks = gridDim.z;
    const int kb0 = int(blockIdx.z) * nsteps / ks, kb1 = (int(blockIdx.z) + 1) * nsteps / ks;

    XStage<BM, 256, W::SPLIT> xs;
    xs.init(a.x, a.ldx, m0, a.M, t);
    auto load_x = [&](int kb) { xs.load(kb); };
    auto stage_x = [&] { xs.template store<W::MIN>(xh, xl, xsum); };

    f4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f4_t{0.f, 0.f, 0.f, 0.f};

    typename W::Regs cur, nxt;
    load_w<T, TL>(a.w, n0 >> 4, ln, kb0, kq, cur);
    load_x(kb0);
    for (int kb = kb0; kb < kb1; ++kb) {
        if (kb != kb0) lds_barrier();  // the previous step's reads of xh / xl / xsum are done
        stage_x();
        lds_barrier();
        if (kb + 1 < kb1) {
            load_w<T, TL>(a.w, n0 >> 4, ln, kb + 1, kq, nxt);
            load_x(kb + 1);
        }
        if constexpr (W::SPLIT) {
            // the block's 8 split-B slices chain in the MFMA's C operand; d once per block
            f4_t cb[MT];
#pragma unroll
            for (int s = 0; s < W::SLICES32; ++s) {
                h8_t bh, bl;
                W::b_split(cur, s, bh, bl);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int xo = (mt * 16 + ln) * kXS + 32 * s + 8 * kq;
                    const h8_t ah = *reinterpret_cast<const h8_t *>(xh + xo), al = *reinterpret_cast<const h8_t *>(xl + xo);
                    cb[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, s ? cb[mt] : f4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    cb[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, cb[mt], 0, 0, 0);
                    cb[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, cb[mt], 0, 0, 0);
                }
            }
            const float d = W::d_of(cur);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[mt][r] = fmaf(d, cb[mt][r], acc[mt][r]);
        } else {
#pragma unroll
            for (int s = 0; s < W::SLICES; ++s) {
                float sc, mn;
                W::scale(cur, s, sc, mn);
                const auto bop = W::b(cur, s);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int xo = (mt * 16 + ln) * kXS + s * W::SK + kq * (W::SK / 4);
                    f4_t tmp = f4_t{0.f, 0.f, 0.f, 0.f};
                    if constexpr (W::SK == 32) {
                        const h8_t ah = *reinterpret_cast<const h8_t *>(xh + xo), al = *reinterpret_cast<const h8_t *>(xl + xo);
                        tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bop, tmp, 0, 0, 0);
                        tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bop, tmp, 0, 0, 0);
                    } else {
                        const h4_t ah = *reinterpret_cast<const h4_t *>(xh + xo), al = *reinterpret_cast<const h4_t *>(xl + xo);
                        tmp = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bop, tmp, 0, 0, 0);
                        tmp = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bop, tmp, 0, 0, 0);
                    }
                    // output rows m = mt 16 + 4 kq + r of this lane; x sums of the slice
                    if constexpr (W::MIN) {
                        const float *xsp = xsum + (s * W::SK / 16) * BM + mt * 16 + 4 * kq;
                        float4 xsv = *reinterpret_cast<const float4 *>(xsp);
                        if constexpr (W::SK == 32) {
                            const float4 x2 = *reinterpret_cast<const float4 *>(xsp + BM);
                            xsv = make_float4(xsv.x + x2.x, xsv.y + x2.y, xsv.z + x2.z, xsv.w + x2.w);
                        }
                        acc[mt][0] = fmaf(sc, tmp[0], fmaf(-mn, xsv.x, acc[mt][0]));
                        acc[mt][1] = fmaf(sc, tmp[1], fmaf(-mn, xsv.y, acc[mt][1]));
                        acc[mt][2] = fmaf(sc, tmp[2], fmaf(-mn, xsv.z, acc[mt][2]));
                        acc[mt][3] = fmaf(sc, tmp[3], fmaf(-mn, xsv.w, acc[mt][3]));
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[mt][r] = fmaf(sc, tmp[r], acc[mt][r]);
                    }
                }
            }
        }
        cur = nxt;
    }
    const int n = n0 + ln;
    if (n >= a.w.N) return;
    if (a.part) {
        float *pp = a.part + size_t(blockIdx.z) * a.M * a.w.N;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + mt * 16 + 4 * kq + r;
                if (m < a.M) pp[size_t(m) * a.w.N + n] = acc[mt][r];
            }
        return;
    }
    const float bv = a.bias ? a.bias[n] : 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + mt * 16 + 4 * kq + r;
            if (m >= a.M) continue;
            float v = acc[mt][r] + bv;
            if (a.R) v += a.R[size_t(m) * a.ldr + n];
            if (a.relu) v = fmaxf(v, 0.f);
            a.y[size_t(m) * a.ldy + n] = v;
        }
}

// y[m][n] = sum_{z < ks} part[z][m][n] (in order) + bias[n] (+ R[m][n]) (relu)
__global__ __launch_bounds__(256) void k_splitk_reduce(const float *part, int ks, int M, int N, const float *bias,
                                                        const float *R, int ldr, int relu, float *y, int ldy) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x, mn = size_t(M) * N;
    if (i >= mn) return;
    const int m = int(i / N), n = int(i % N);
    float v = 0.f;
    for (int z0 = 0; z0 < ks; z0 += 8) {
        float p8[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) p8[u] = z0 + u < ks ? part[size_t(z0 + u) * mn + i] : 0.f;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z0 + u < ks) v = (z0 + u == 0) ? p8[u] : v + p8[u];
    }
    if (bias) v += bias[n];
    if (R) v += R[size_t(m) * ldr + n];
    if (relu) v = fmaxf(v, 0.f);
    y[size_t(m) * ldy + n] = v;
}

// ------------------------------------------------------------- wide tiles
//
// For large N at M > 32 (the LM head and FFN of batched decode, encoder prefill):
// 8 waves, each owning WT 16-row tiles of W, so a workgroup covers 128 WT rows of
// W and one staging of X per K step (f32 -> f16 hi/lo in LDS, x sums) serves
// 2 WT times more rows than in k_mfma.  A wave reads each X fragment from LDS once
// per slice and uses it for its WT tiles.
constexpr int kWWaves = 8;

template <int BM>
constexpr size_t mfma_w_lds() {
    return size_t(2) * BM * kXS * sizeof(_Float16) + size_t(16) * BM * sizeof(float);
}

// MODE 0 stores Y (or split-K partials); MODE 1 (the greedy LM head of 33..64 rows) keeps
// a (value, lowest index) argmax per X row and workgroup instead (gridDim.y = z = 1).
template <int T, int BM, int WT, bool TL, int MODE = 0>
__global__ __launch_bounds__(512) void k_mfma_w(MfmaArgs a) {
    using W = MW<T>;
    constexpr int MT = BM / 16;
    constexpr int NTH = kWWaves * 64;
    extern __shared__ __align__(16) unsigned char wlds[];
    _Float16 *xh = reinterpret_cast<_Float16 *>(wlds);
    _Float16 *xl = xh + BM * kXS;
    float *xsum = reinterpret_cast<float *>(xl + BM * kXS);  // [16-slice][m]
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int kq = lane >> 4, ln = lane & 15;
    const int n0 = blockIdx.x * (kWWaves * 16 * WT) + w * 16 * WT;
    const int m0 = blockIdx.y * BM;
    const int nsteps = a.w.K / kStep, ks = gridDim.z;
    const int kb0 = int(blockIdx.z) * nsteps / ks, kb1 = (int(blockIdx.z) + 1) * nsteps / ks;

    XStage<BM, NTH, W::SPLIT> xs;
    xs.init(a.x, a.ldx, m0, a.M, t);
    auto load_x = [&](int kb) { xs.load(kb); };
    auto stage_x = [&] { xs.template store<W::MIN>(xh, xl, xsum); };

    f4_t acc[WT][MT];
#pragma unroll
    for (int j = 0; j < WT; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[j][mt] = f4_t{0.f, 0.f, 0.f, 0.f};

    typename W::Regs cur[WT], nxt[WT];
#pragma unroll
    for (int j = 0; j < WT; ++j) load_w<T, TL>(a.w, (n0 >> 4) + j, ln, kb0, kq, cur[j]);
    load_x(kb0);
    for (int kb = kb0; kb < kb1; ++kb) {
        if (kb != kb0) lds_barrier();  // the previous step's reads of xh / xl / xsum are done
        stage_x();
        lds_barrier();
        if (kb + 1 < kb1) {
#pragma unroll
            for (int j = 0; j < WT; ++j) load_w<T, TL>(a.w, (n0 >> 4) + j, ln, kb + 1, kq, nxt[j]);
            load_x(kb + 1);
        }
        if constexpr (W::SPLIT) {
            // the block's 8 split-B slices chain in the MFMA's C operand; d once per block
            f4_t cb[WT][MT];
            // A fragments of slice s + 1 are read from LDS while slice s runs on the MFMA
            h8_t ahs[2][MT], als[2][MT];
            auto read_a = [&](int s, h8_t (&ah)[MT], h8_t (&al)[MT]) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int xo = (mt * 16 + ln) * kXS + 32 * s + 8 * kq;
                    ah[mt] = *reinterpret_cast<const h8_t *>(xh + xo);
                    al[mt] = *reinterpret_cast<const h8_t *>(xl + xo);
                }
            };
            read_a(0, ahs[0], als[0]);
#pragma unroll
            for (int s = 0; s < W::SLICES32; ++s) {
                if (s + 1 < W::SLICES32) read_a(s + 1, ahs[(s + 1) & 1], als[(s + 1) & 1]);
                h8_t bh[WT], bl[WT];
#pragma unroll
                for (int j = 0; j < WT; ++j) W::b_split(cur[j], s, bh[j], bl[j]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const h8_t ah = ahs[s & 1][mt], al = als[s & 1][mt];
#pragma unroll
                    for (int j = 0; j < WT; ++j)
                        cb[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[j], s ? cb[j][mt] : f4_t{0.f, 0.f, 0.f, 0.f},
                                                                          0, 0, 0);
#pragma unroll
                    for (int j = 0; j < WT; ++j) cb[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[j], cb[j][mt], 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < WT; ++j) cb[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[j], cb[j][mt], 0, 0, 0);
                }
            }
#pragma unroll
            for (int j = 0; j < WT; ++j) {
                const float d = W::d_of(cur[j]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[j][mt][r] = fmaf(d, cb[j][mt][r], acc[j][mt][r]);
            }
        } else {
#pragma unroll
            for (int s = 0; s < W::SLICES; ++s) {
                float sc[WT], mn[WT];
                decltype(W::b(cur[0], 0)) bop[WT];
#pragma unroll
                for (int j = 0; j < WT; ++j) {
                    W::scale(cur[j], s, sc[j], mn[j]);
                    bop[j] = W::b(cur[j], s);
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int xo = (mt * 16 + ln) * kXS + s * W::SK + kq * (W::SK / 4);
                    float4 xsv = make_float4(0.f, 0.f, 0.f, 0.f);
                    if constexpr (W::MIN) {
                        const float *xsp = xsum + (s * W::SK / 16) * BM + mt * 16 + 4 * kq;
                        xsv = *reinterpret_cast<const float4 *>(xsp);
                        if constexpr (W::SK == 32) {
                            const float4 x2 = *reinterpret_cast<const float4 *>(xsp + BM);
                            xsv = make_float4(xsv.x + x2.x, xsv.y + x2.y, xsv.z + x2.z, xsv.w + x2.w);
                        }
                    }
                    // acc += sc tmp (- mn xsum for the formats with mins)
                    auto scale_add = [&](f4_t &a4, const f4_t &tmp, float scj, float mnj) {
                        if constexpr (W::MIN) {
                            a4[0] = fmaf(scj, tmp[0], fmaf(-mnj, xsv.x, a4[0]));
                            a4[1] = fmaf(scj, tmp[1], fmaf(-mnj, xsv.y, a4[1]));
                            a4[2] = fmaf(scj, tmp[2], fmaf(-mnj, xsv.z, a4[2]));
                            a4[3] = fmaf(scj, tmp[3], fmaf(-mnj, xsv.w, a4[3]));
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r) a4[r] = fmaf(scj, tmp[r], a4[r]);
                        }
                    };
                    if constexpr (W::SK == 32) {
                        const h8_t ah = *reinterpret_cast<const h8_t *>(xh + xo), al = *reinterpret_cast<const h8_t *>(xl + xo);
#pragma unroll
                        for (int j = 0; j < WT; ++j) {
                            f4_t tmp = f4_t{0.f, 0.f, 0.f, 0.f};
                            tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bop[j], tmp, 0, 0, 0);
                            tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bop[j], tmp, 0, 0, 0);
                            scale_add(acc[j][mt], tmp, sc[j], mn[j]);
                        }
                    } else {
                        const h4_t ah = *reinterpret_cast<const h4_t *>(xh + xo), al = *reinterpret_cast<const h4_t *>(xl + xo);
#pragma unroll
                        for (int j = 0; j < WT; ++j) {
                            f4_t tmp = f4_t{0.f, 0.f, 0.f, 0.f};
                            tmp = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bop[j], tmp, 0, 0, 0);
                            tmp = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bop[j], tmp, 0, 0, 0);
                            scale_add(acc[j][mt], tmp, sc[j], mn[j]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < WT; ++j) cur[j] = nxt[j];
    }
    if constexpr (MODE == 1) {
        // lane (kq, ln) holds rows mt 16 + 4 kq + r of columns n0 + 16 j + ln: its best over
        // its WT columns, then over the 16 lanes of the row group (DPP), then over the
        // waves (LDS; every wave's reads of the staged X are done first)
        float best[MT][4];
        uint32_t bidx[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                best[mt][r] = -INFINITY;
                bidx[mt][r] = 0xffffffffu;
            }
#pragma unroll
        for (int j = 0; j < WT; ++j) {
            const int n = n0 + 16 * j + ln;
            if (n >= a.w.N || n == a.mask_id) continue;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) argmax_merge(best[mt][r], bidx[mt][r], acc[j][mt][r], uint32_t(n));
        }
        __syncthreads();
        float *mv = reinterpret_cast<float *>(wlds);                     // [waves][BM]
        uint32_t *mi = reinterpret_cast<uint32_t *>(mv + kWWaves * BM);  // [waves][BM]
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = best[mt][r];
                uint32_t i = bidx[mt][r];
                argmax_merge(v, i, dpp_mov<kDppXor1>(v), dpp_mov<kDppXor1>(i));
                argmax_merge(v, i, dpp_mov<kDppXor2>(v), dpp_mov<kDppXor2>(i));
                argmax_merge(v, i, dpp_mov<kDppHalfMirror>(v), dpp_mov<kDppHalfMirror>(i));
                argmax_merge(v, i, dpp_mov<kDppMirror>(v), dpp_mov<kDppMirror>(i));
                if (ln == 0) {
                    mv[w * BM + mt * 16 + 4 * kq + r] = v;
                    mi[w * BM + mt * 16 + 4 * kq + r] = i;
                }
            }
        __syncthreads();
        if (t < BM && m0 + t < a.M) {  // ties -> the lowest index, so the merge order is free
            float v = mv[t];
            uint32_t i = mi[t];
#pragma unroll
            for (int w2 = 1; w2 < kWWaves; ++w2) argmax_merge(v, i, mv[w2 * BM + t], mi[w2 * BM + t]);
            a.pv[size_t(m0 + t) * a.parts + blockIdx.x] = v;
            a.pi[size_t(m0 + t) * a.parts + blockIdx.x] = i;
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < WT; ++j) {
        const int n = n0 + 16 * j + ln;
        if (n >= a.w.N) continue;
        if (a.part) {
            float *pp = a.part + size_t(blockIdx.z) * a.M * a.w.N;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + mt * 16 + 4 * kq + r;
                    if (m < a.M) pp[size_t(m) * a.w.N + n] = acc[j][mt][r];
                }
            continue;
        }
        const float bv = a.bias ? a.bias[n] : 0.f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + mt * 16 + 4 * kq + r;
                if (m >= a.M) continue;
                float v = acc[j][mt][r] + bv;
                if (a.R) v += a.R[size_t(m) * a.ldr + n];
                if (a.relu) v = fmaxf(v, 0.f);
                a.y[size_t(m) * a.ldy + n] = v;
            }
    }
}

// W tiles per wave of the wide kernel for (N, M), 0: use k_mfma.  Wide tiles pay
// off once X (M > 32 rows) is re-staged by many tiles and enough workgroups remain:
// from 96 wide workgroups (config 4's encoder QKV, N = 3072 at 13 row tiles: 105.9 us on
// k_mfma -> 35 us; at 48 the K = 4096 FFN-down switches too and slows, 37.4 -> 43.6 us).
int wide_wt(int N, int M) {
    if (M <= 32) return 0;
    const int gy = (M + 63) / 64;
    // WT = 4 (512 rows) would need more than the 256 registers a wave of a
    // 512-thread workgroup can hold (spills), so 2 (256 rows)
    return size_t((N + 255) / 256) * gy >= 96 ? 2 : 0;
}

template <int T, int BM, int WT, bool TL, int MODE = 0>
hipError_t launch_w_t(const MfmaArgs &a, int M, int ks, hipStream_t st) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_mfma_w<T, BM, WT, TL, MODE>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       int(mfma_w_lds<BM>()));
    if (attr != hipSuccess) return attr;
    const int gx = (a.w.N + 128 * WT - 1) / (128 * WT);
    hipLaunchKernelGGL((k_mfma_w<T, BM, WT, TL, MODE>), dim3(gx, (M + BM - 1) / BM, ks), dim3(kWWaves * 64),
                       mfma_w_lds<BM>(), st, a);
    return hipGetLastError();
}

template <int T, bool TL>
hipError_t launch_tl(const MfmaArgs &a, int M, int ks, hipStream_t st) {
    if (wide_wt(a.w.N, M) == 2) return launch_w_t<T, 64, 2, TL>(a, M, ks, st);
    const int gx = (a.w.N + kTileN - 1) / kTileN;
    if (M <= 16) {
        hipLaunchKernelGGL((k_mfma<T, 16, TL>), dim3(gx, (M + 15) / 16, ks), dim3(256), 0, st, a);
    } else if (M <= 32) {
        hipLaunchKernelGGL((k_mfma<T, 32, TL>), dim3(gx, 1, ks), dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL((k_mfma<T, 64, TL>), dim3(gx, (M + 63) / 64, ks), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

// q6_K / q4_K with its tile-major copy reads that copy
template <int T>
hipError_t launch(const MfmaArgs &a, int M, int ks, hipStream_t st) {
    if constexpr (T == GGML_Q6_K || T == GGML_Q4_K) {
        if (a.w.t) return launch_tl<T, true>(a, M, ks, st);
    }
    return launch_tl<T, false>(a, M, ks, st);
}

// Split-K reduction fused with the decoder's residual add and the next LayerNorm
// (src/model.rs:183-187): y = sum_z part[z][m] (in z order) + bias; x[m] += y;
// h[m] = LayerNorm(x[m]) with biased variance (f64 statistics).  One workgroup of 256
// threads per row, each thread on float4 slots t + 256 c; N <= 4096, N % 4 == 0.
__global__ __launch_bounds__(256) void k_splitk_residual_ln(const float *part, int ks, int M, int N,
                                                             const float *bias, float *x, const float *g,
                                                             const float *b, float eps, float *h) {
    __shared__ double red[8];
    const int m = blockIdx.x;
    const size_t mn = size_t(M) * N, off = size_t(m) * N;
    float4 *xr = reinterpret_cast<float4 *>(x + off);
    auto form = [&](int f) {
        // the partials requested eight at a time, then added in z order
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int z0 = 0; z0 < ks; z0 += 8) {
            float4 p8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                p8[u] = z0 + u < ks ? ld4(part + size_t(z0 + u) * mn + off, f) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (z0 + u < ks) {
                    if (z0 + u == 0) y = p8[u];
                    else add4(y, p8[u]);
                }
        }
        if (bias) add4(y, ld4(bias, f));
        float4 v = xr[f];
        add4(v, y);
        return v;
    };
    workgroup_row_layernorm<4>(N, form, [&](int f, const float4 &v) { xr[f] = v; }, g, b, eps, h + off, red);
}

// Split-K reduction of the fused QKV projection written straight into q [M][d] and
// the caches at slot *step (kernels/malaga.cu:142-154): f16 (rounded to nearest even) or
// f32 (the generic path's caches).
__device__ __forceinline__ void store_kv(__half *p, float v) { *p = __float2half(v); }
__device__ __forceinline__ void store_kv(float *p, float v) { *p = v; }

template <typename KT>
__global__ __launch_bounds__(256) void k_splitk_qkv(const float *part, int ks, int M, int d, const float *bias, int H,
                                                     int hd, int slots, const uint32_t *step, float *q, KT *kc,
                                                     KT *vc) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x, N = size_t(3) * d, mn = size_t(M) * N;
    if (i >= mn) return;
    const int m = int(i / N), c = int(i % N);
    float v = 0.f;
    for (int z0 = 0; z0 < ks; z0 += 8) {
        float p8[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) p8[u] = z0 + u < ks ? part[size_t(z0 + u) * mn + i] : 0.f;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z0 + u < ks) v = (z0 + u == 0) ? p8[u] : v + p8[u];
    }
    if (bias) v += bias[c];
    if (c < d) {
        q[size_t(m) * d + c] = v;
    } else {
        const int cc = c < 2 * d ? c - d : c - 2 * d;
        const size_t o = ((size_t(m) * H + cc / hd) * slots + *step) * hd + cc % hd;
        store_kv((c < 2 * d ? kc : vc) + o, v);
    }
}

// K splits that bring the grid to about one workgroup per CU, within the workspace
int split_k(const DevMatrix &w, int M, size_t ws_bytes) {
    const int wt = wide_wt(w.N, M);
    const int gx = wt ? (w.N + 128 * wt - 1) / (128 * wt) : (w.N + kTileN - 1) / kTileN;
    const int bm = M <= 16 ? 16 : M <= 32 ? 32 : 64;
    const int base = gx * ((M + bm - 1) / bm), nsteps = w.K / kStep;
    int ks = base >= 256 ? 1 : std::min(nsteps, (256 + base - 1) / base);
    while (ks > 1 && size_t(ks) * M * w.N * sizeof(float) > ws_bytes) --ks;
    return ks;
}

// ---------------------------------------------------------------- resident X
//
// Decode batches (M <= 32) with K small enough that all of X fits in LDS as hi/lo
// f16 (BM * K * 4 bytes <= ~140 KB): one persistent workgroup of 8 waves per CU
// stages X once, then every wave streams 16-row tiles of W (tile t, t + waves, ...)
// with the next (tile, K-step) in flight in registers.  No split K, no reduction
// kernel, and X is read from HBM/L2 once per workgroup instead of once per tile.
// MODE 0 stores Y (bias, residual, ReLU); MODE 1 keeps a running argmax per X row
// (the greedy LM head) and writes one partial per workgroup (its waves' merged in LDS).

constexpr int kRxWaves = 8;
constexpr int kRxDepth = 2;  // (group, K-step) jobs of W in flight per wave
// 16-row tiles of W per job (reuse of each X fragment), sized to the registers a
// type's raw K step needs; q6_K issues 14 loads per tile and K step, and a wave
// tracks at most 63 outstanding loads (kRxDepth x tiles x loads must stay below,
// or every job waits for all loads in flight)
template <int T>
constexpr int rx_nt() { return T == GGML_F16 ? 1 : (T == GGML_Q8_0 || T == GGML_Q6_K) ? 2 : 4; }
constexpr size_t kRxMaxLds = 150 * 1024;

struct RxArgs {
    WPtr w;
    const float *x;
    int ldx, M;
    float *y;
    int ldy;
    const float *bias, *R;
    int ldr, relu;
    int mask_id;      // MODE 1: row index never selected (-1: none)
    float *pv;        // MODE 1: partials [M][parts]
    uint32_t *pi;
    int parts;
};

// halves per staged X row: 8 mod 64 dwords, where the A reads (16 rows x 4 k-groups of
// 16 bytes) meet no bank conflict (K + 8: 5.4 M conflict cycles per LM-head launch)
__host__ __device__ constexpr int rx_stride(int K) { return K + 16; }

size_t rx_lds_bytes(int BM, int K) {
    return size_t(BM) * rx_stride(K) * 2 * sizeof(_Float16) + size_t(K / 16) * BM * sizeof(float);
}

template <int T, int BM, int MODE, bool TL>
__global__ __launch_bounds__(kRxWaves * 64) void k_mfma_rx(RxArgs a) {
    using W = MW<T>;
    constexpr int MT = BM / 16;
    constexpr int kRxNT = rx_nt<T>();
    extern __shared__ __align__(16) unsigned char rx_lds[];
    const int K = a.w.K, XS = rx_stride(K);
    _Float16 *xh = reinterpret_cast<_Float16 *>(rx_lds);
    _Float16 *xl = xh + BM * XS;
    float *xsum = reinterpret_cast<float *>(xl + BM * XS);  // [K / 16][BM]
    const int t = threadIdx.x, lane = t & 63;
    const int kq = lane >> 4, ln = lane & 15;
    const int nsteps = K / kStep;
    const int ngroups = (a.w.N + 16 * kRxNT - 1) / (16 * kRxNT);  // groups of kRxNT 16-row tiles
    // a scalar: the job loop's bounds stay uniform (no divergent load paths)
    const int gw = __builtin_amdgcn_readfirstlane(blockIdx.x * kRxWaves + (t >> 6)), nw = gridDim.x * kRxWaves;
    const int njobs = gw < ngroups ? ((ngroups - 1 - gw) / nw + 1) * nsteps : 0;  // (group, step) pairs of this wave

    typename W::Regs ring[kRxDepth][kRxNT];
    auto job_base = [&](int j) { return (gw + (j / nsteps) * nw) * 16 * kRxNT; };
    auto load_job = [&](int j, typename W::Regs (&r)[kRxNT]) {
#pragma unroll
        for (int nt = 0; nt < kRxNT; ++nt) load_w<T, TL>(a.w, (job_base(j) >> 4) + nt, ln, j % nsteps, kq, r[nt]);
    };

    // stage X: chunks of 8 values, one 16-byte store each (consecutive lanes: consecutive
    // chunks of a row, so a store of 16 lanes covers 256 contiguous bytes of LDS: no bank
    // conflicts), up to 4 per thread in flight.  Chunk c of a row holds x[8 c .. 8 c + 7], or
    // for split-B types the two 4-value groups split_pos puts there.  BM K / 8 is a multiple
    // of the 512 threads, so every lane runs the same trips (the DPP sums below need them all).
    {
        const int cpr = K / 8, nch = BM * cpr;
        auto koff = [](int c, int half) {
            if constexpr (W::SPLIT) return 32 * (c >> 2) + 16 * half + 4 * (c & 3);
            else return 8 * c + 4 * half;
        };
        for (int c0 = t; c0 < nch; c0 += kRxWaves * 64 * 4) {
            float4 v[4][2];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = c0 + u * kRxWaves * 64;
                const int m = c / cpr, cc = c % cpr;
                const bool ok = c < nch && m < a.M;
                const float *src = a.x + size_t(ok ? m : 0) * a.ldx;
#pragma unroll
                for (int f = 0; f < 2; ++f)
                    v[u][f] = ok ? *reinterpret_cast<const float4 *>(src + koff(cc, f)) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = c0 + u * kRxWaves * 64;
                if (c >= nch) break;  // the same trips in every lane
                const int m = c / cpr, cc = c % cpr;
                const float e[8] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w,
                                    v[u][1].x, v[u][1].y, v[u][1].z, v[u][1].w};
                h8_t hv, lv;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    hv[i] = _Float16(e[i]);
                    lv[i] = _Float16(e[i] - float(hv[i]));
                }
                *reinterpret_cast<h8_t *>(xh + m * XS + 8 * cc) = hv;
                *reinterpret_cast<h8_t *>(xl + m * XS + 8 * cc) = lv;
                if constexpr (W::MIN) {  // 16-value sums: this chunk and the next (lane t ^ 1)
                    float sm = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
                    sm += dpp_mov<kDppXor1>(sm);
                    if (!(cc & 1)) xsum[(cc >> 1) * BM + m] = sm;
                }
            }
        }
    }
    __syncthreads();
    // the first kRxDepth (group, K-step) jobs of W: requested once X is staged, so that
    // the job loop is entered with the same loads in flight as on every later trip
    // (requested before the staging, they made the compiler wait for every load at the
    // top of each job: 2 of the ring's jobs in flight became 0)
    // (unconditional: a job past this wave's last reads a clamped row and is never used;
    // a skipped request would leave the compiler unsure how many loads follow each one)
#pragma unroll
    for (int u = 0; u < kRxDepth; ++u) {
        load_job(u, ring[u]);
        __builtin_amdgcn_sched_barrier(0);  // jobs requested in order
    }

    f4_t acc[MT][kRxNT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < kRxNT; ++nt) acc[mt][nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    float best[MT][4];
    uint32_t bidx[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            best[mt][r] = -INFINITY;
            bidx[mt][r] = 0xffffffffu;
        }

    // job j uses ring slot j % kRxDepth, refilled with job j + kRxDepth once consumed;
    // each X fragment read from LDS feeds kRxNT tiles of W
    auto job = [&](int j, const typename W::Regs (&cur)[kRxNT]) {
        const int kb = j % nsteps;
        if constexpr (W::SPLIT) {
            // the block's 8 split-B slices chain in the MFMA's C operand; d once per block
            f4_t cb[MT][kRxNT];
            // A fragments of slice s + 1 are read from LDS while slice s runs on the MFMA
            h8_t ahs[2][MT], als[2][MT];
            auto read_a = [&](int s, h8_t (&ah)[MT], h8_t (&al)[MT]) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int xo = (mt * 16 + ln) * XS + kb * kStep + 32 * s + 8 * kq;
                    ah[mt] = *reinterpret_cast<const h8_t *>(xh + xo);
                    al[mt] = *reinterpret_cast<const h8_t *>(xl + xo);
                }
            };
            read_a(0, ahs[0], als[0]);
#pragma unroll
            for (int s = 0; s < W::SLICES32; ++s) {
                if (s + 1 < W::SLICES32) read_a(s + 1, ahs[(s + 1) & 1], als[(s + 1) & 1]);
                h8_t bh[kRxNT], bl[kRxNT];
#pragma unroll
                for (int nt = 0; nt < kRxNT; ++nt) W::b_split(cur[nt], s, bh[nt], bl[nt]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const h8_t ah = ahs[s & 1][mt], al = als[s & 1][mt];
#pragma unroll
                    for (int nt = 0; nt < kRxNT; ++nt)
                        cb[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            ah, bh[nt], s ? cb[mt][nt] : f4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                    for (int nt = 0; nt < kRxNT; ++nt)
                        cb[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[nt], cb[mt][nt], 0, 0, 0);
#pragma unroll
                    for (int nt = 0; nt < kRxNT; ++nt)
                        cb[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[nt], cb[mt][nt], 0, 0, 0);
                }
            }
#pragma unroll
            for (int nt = 0; nt < kRxNT; ++nt) {
                const float d = W::d_of(cur[nt]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[mt][nt][r] = fmaf(d, cb[mt][nt][r], acc[mt][nt][r]);
            }
        } else {
#pragma unroll
            for (int s = 0; s < W::SLICES; ++s) {
                float sc[kRxNT], mn[kRxNT];
                decltype(W::b(cur[0], s)) bop[kRxNT];
#pragma unroll
                for (int nt = 0; nt < kRxNT; ++nt) {
                    W::scale(cur[nt], s, sc[nt], mn[nt]);
                    bop[nt] = W::b(cur[nt], s);
                }
                const int kx = kb * kStep + s * W::SK;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int xo = (mt * 16 + ln) * XS + kx + kq * (W::SK / 4);
                    const float *xsp = xsum + (kx >> 4) * BM + mt * 16 + 4 * kq;
                    float4 xsv = make_float4(0.f, 0.f, 0.f, 0.f);
                    if constexpr (W::MIN) {
                        xsv = *reinterpret_cast<const float4 *>(xsp);
                        if constexpr (W::SK == 32) {
                            const float4 x2 = *reinterpret_cast<const float4 *>(xsp + BM);
                            xsv = make_float4(xsv.x + x2.x, xsv.y + x2.y, xsv.z + x2.z, xsv.w + x2.w);
                        }
                    }
                    if constexpr (W::SK == 32) {
                        const h8_t ah = *reinterpret_cast<const h8_t *>(xh + xo), al = *reinterpret_cast<const h8_t *>(xl + xo);
#pragma unroll
                        for (int nt = 0; nt < kRxNT; ++nt) {
                            f4_t tmp = f4_t{0.f, 0.f, 0.f, 0.f};
                            tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bop[nt], tmp, 0, 0, 0);
                            tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bop[nt], tmp, 0, 0, 0);
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                acc[mt][nt][r] = W::MIN ? fmaf(sc[nt], tmp[r], fmaf(-mn[nt], (&xsv.x)[r], acc[mt][nt][r]))
                                                        : fmaf(sc[nt], tmp[r], acc[mt][nt][r]);
                        }
                    } else {
                        const h4_t ah = *reinterpret_cast<const h4_t *>(xh + xo), al = *reinterpret_cast<const h4_t *>(xl + xo);
#pragma unroll
                        for (int nt = 0; nt < kRxNT; ++nt) {
                            f4_t tmp = f4_t{0.f, 0.f, 0.f, 0.f};
                            tmp = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bop[nt], tmp, 0, 0, 0);
                            tmp = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bop[nt], tmp, 0, 0, 0);
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                acc[mt][nt][r] = W::MIN ? fmaf(sc[nt], tmp[r], fmaf(-mn[nt], (&xsv.x)[r], acc[mt][nt][r]))
                                                        : fmaf(sc[nt], tmp[r], acc[mt][nt][r]);
                        }
                    }
                }
            }
        }
        if (kb == nsteps - 1) {  // group done
#pragma unroll
            for (int nt = 0; nt < kRxNT; ++nt) {
                const int n = job_base(j) + nt * 16 + ln;
                if (n < a.w.N) {
                    // MODE 1 (the tied LM head) has no bias: no global load in this
                    // epilogue, which would make every later job wait for all loads
                    float bv = 0.f;
                    if constexpr (MODE == 0) bv = a.bias ? a.bias[n] : 0.f;
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int m = mt * 16 + 4 * kq + r;
                            float v = acc[mt][nt][r] + bv;
                            if constexpr (MODE == 0) {
                                if (m < a.M) {
                                    if (a.R) v += a.R[size_t(m) * a.ldr + n];
                                    if (a.relu) v = fmaxf(v, 0.f);
                                    a.y[size_t(m) * a.ldy + n] = v;
                                }
                            } else {
                                if (n != a.mask_id) argmax_merge(best[mt][r], bidx[mt][r], v, uint32_t(n));
                            }
                        }
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = f4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    // Main loop: every job is followed by its slot's refill.  The last jobs run in a
    // separate tail, so that no job in the main loop follows a skipped refill: the
    // compiler would then merge the two load states and wait for every load in
    // flight (the refills included) at the top of each job.
    int j0 = 0;
    for (; j0 + 2 * kRxDepth <= njobs; j0 += kRxDepth) {
#pragma unroll
        for (int u = 0; u < kRxDepth; ++u) {
            job(j0 + u, ring[u]);
            __builtin_amdgcn_sched_barrier(0);
            load_job(j0 + u + kRxDepth, ring[u]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    for (; j0 < njobs; j0 += kRxDepth) {
#pragma unroll
        for (int u = 0; u < kRxDepth; ++u) {
            const int j = j0 + u;
            if (j >= njobs) break;  // wave-uniform
            job(j, ring[u]);
            if (j + kRxDepth < njobs) load_job(j + kRxDepth, ring[u]);
        }
    }
    if constexpr (MODE == 1) {
        // lanes 16 kq .. 16 kq + 15 hold the same X rows: reduce within each 16-lane row,
        // then over the workgroup's waves (LDS; the staged X is no longer read), so the
        // finalize merges one partial per workgroup and row
        __syncthreads();  // every wave's last reads of the staged X are done
        float *mv = reinterpret_cast<float *>(rx_lds);                  // [kRxWaves][BM]
        uint32_t *mi = reinterpret_cast<uint32_t *>(mv + kRxWaves * BM);  // [kRxWaves][BM]
        const int wv = t >> 6;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = best[mt][r];
                uint32_t i = bidx[mt][r];
                argmax_merge(v, i, dpp_mov<kDppXor1>(v), dpp_mov<kDppXor1>(i));
                argmax_merge(v, i, dpp_mov<kDppXor2>(v), dpp_mov<kDppXor2>(i));
                argmax_merge(v, i, dpp_mov<kDppHalfMirror>(v), dpp_mov<kDppHalfMirror>(i));
                argmax_merge(v, i, dpp_mov<kDppMirror>(v), dpp_mov<kDppMirror>(i));
                const int m = mt * 16 + 4 * kq + r;
                if (ln == 0) {
                    mv[wv * BM + m] = v;
                    mi[wv * BM + m] = i;
                }
            }
        __syncthreads();
        if (t < BM && t < a.M) {  // ties -> the lowest index, so the order of the merge is free
            float v = mv[t];
            uint32_t i = mi[t];
#pragma unroll
            for (int w2 = 1; w2 < kRxWaves; ++w2) argmax_merge(v, i, mv[w2 * BM + t], mi[w2 * BM + t]);
            a.pv[size_t(t) * a.parts + blockIdx.x] = v;
            a.pi[size_t(t) * a.parts + blockIdx.x] = i;
        }
    }
}

// Dynamic LDS beyond 64 KB needs the kernel attribute raised once.
template <int T, int BM, int MODE, bool TL>
hipError_t launch_rx_bm(const RxArgs &a, int grid, hipStream_t st) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_mfma_rx<T, BM, MODE, TL>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(kRxMaxLds));
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((k_mfma_rx<T, BM, MODE, TL>), dim3(grid), dim3(kRxWaves * 64), rx_lds_bytes(BM, a.w.K), st,
                       a);
    return hipGetLastError();
}

template <int T, int MODE, bool TL>
hipError_t launch_rx_tl(const RxArgs &a, int M, int grid, hipStream_t st) {
    return M <= 16 ? launch_rx_bm<T, 16, MODE, TL>(a, grid, st) : launch_rx_bm<T, 32, MODE, TL>(a, grid, st);
}

template <int T, int MODE>
hipError_t launch_rx(const RxArgs &a, int M, int grid, hipStream_t st) {
    if constexpr (T == GGML_Q6_K || T == GGML_Q4_K) {
        if (a.w.t) return launch_rx_tl<T, MODE, true>(a, M, grid, st);
    }
    return launch_rx_tl<T, MODE, false>(a, M, grid, st);
}

int rx_nt_of(uint32_t t) {
    switch (t) {
    case GGML_F16: return rx_nt<GGML_F16>();
    case GGML_Q8_0: return rx_nt<GGML_Q8_0>();
    case GGML_Q6_K: return rx_nt<GGML_Q6_K>();
    case GGML_Q5_K: return rx_nt<GGML_Q5_K>();
    default: return rx_nt<GGML_Q4_K>();
    }
}

int rx_grid(const DevMatrix &w, int M) {
    const int bm = M <= 16 ? 16 : 32;
    const size_t lds = rx_lds_bytes(bm, w.K);
    const int per_cu = lds * 2 <= 160 * 1024 ? 2 : 1;
    const int nt = rx_nt_of(w.type);
    const int groups = (w.N + 16 * nt - 1) / (16 * nt);
    const int waves = std::min(groups, 256 * per_cu * kRxWaves);
    return (waves + kRxWaves - 1) / kRxWaves;
}

}  // namespace

bool gemm_mfma_supported(const DevMatrix &w) {
    const bool type_ok = w.type == GGML_Q4_K || w.type == GGML_Q5_K || w.type == GGML_Q6_K ||
                         w.type == GGML_Q8_0 || w.type == GGML_F16;
    return type_ok && w.K % kStep == 0 && w.N > 0;
}

bool gemm_rx_supported(const DevMatrix &w, int M) {
    return gemm_mfma_supported(w) && M >= 1 && M <= 32 && rx_lds_bytes(M <= 16 ? 16 : 32, w.K) <= kRxMaxLds;
}

// Stored products take the resident-X kernel only when W is large enough to keep
// every CU busy (staging X per workgroup is then amortised); smaller matrices use
// the split-K tile kernel.
constexpr int kRxMinRows = 65536;

namespace {
template <int MODE>
hipError_t run_rx(const DevMatrix &w, RxArgs &a, int M, int grid, hipStream_t st) {
    switch (w.type) {
    case GGML_Q4_K: return launch_rx<GGML_Q4_K, MODE>(a, M, grid, st);
    case GGML_Q5_K: return launch_rx<GGML_Q5_K, MODE>(a, M, grid, st);
    case GGML_Q6_K: return launch_rx<GGML_Q6_K, MODE>(a, M, grid, st);
    case GGML_Q8_0: return launch_rx<GGML_Q8_0, MODE>(a, M, grid, st);
    case GGML_F16: return launch_rx<GGML_F16, MODE>(a, M, grid, st);
    default: return hipErrorInvalidValue;
    }
}
RxArgs rx_args(const DevMatrix &w, const float *X, int ldx, int M) {
    RxArgs a{};
    a.w = wptr_of(w);
    a.x = X;
    a.ldx = ldx;
    a.M = M;
    a.mask_id = -1;
    return a;
}
}  // namespace

// 33..64 rows: the wide-tile kernel with the argmax epilogue (X staged per K step)
namespace {
constexpr int kWArgmaxMaxRows = 64;
bool w_argmax_rows(const DevMatrix &w, int M) {
    return !gemm_rx_supported(w, M) && gemm_mfma_supported(w) && M > 32 && M <= kWArgmaxMaxRows;
}
int w_argmax_grid(const DevMatrix &w) { return (w.N + 256 - 1) / 256; }  // WT = 2: 256 rows of W per workgroup

template <int T>
hipError_t launch_w_argmax(const MfmaArgs &a, int M, hipStream_t st) {
    if constexpr (T == GGML_Q6_K || T == GGML_Q4_K) {
        if (a.w.t) return launch_w_t<T, 64, 2, true, 1>(a, M, 1, st);
    }
    return launch_w_t<T, 64, 2, false, 1>(a, M, 1, st);
}
}  // namespace

bool gemm_argmax_supported(const DevMatrix &w, int M) { return gemm_rx_supported(w, M) || w_argmax_rows(w, M); }

// one partial per workgroup
int gemm_argmax_parts(const DevMatrix &w, int M) { return w_argmax_rows(w, M) ? w_argmax_grid(w) : rx_grid(w, M); }

hipError_t gemm_argmax(const DevMatrix &w, const float *X, int ldx, int M, int mask_id, float *pv, uint32_t *pi,
                       int *parts, hipStream_t st) {
    if (!gemm_argmax_supported(w, M) || ldx % 4 || reinterpret_cast<uintptr_t>(X) % 16) return hipErrorInvalidValue;
    if (w_argmax_rows(w, M)) {
        MfmaArgs a{};
        a.w = wptr_of(w);
        a.x = X;
        a.ldx = ldx;
        a.M = M;
        a.mask_id = mask_id;
        a.pv = pv;
        a.pi = pi;
        a.parts = w_argmax_grid(w);
        *parts = a.parts;
        switch (w.type) {
        case GGML_Q4_K: return launch_w_argmax<GGML_Q4_K>(a, M, st);
        case GGML_Q5_K: return launch_w_argmax<GGML_Q5_K>(a, M, st);
        case GGML_Q6_K: return launch_w_argmax<GGML_Q6_K>(a, M, st);
        case GGML_Q8_0: return launch_w_argmax<GGML_Q8_0>(a, M, st);
        case GGML_F16: return launch_w_argmax<GGML_F16>(a, M, st);
        default: return hipErrorInvalidValue;
        }
    }
    RxArgs a = rx_args(w, X, ldx, M);
    a.mask_id = mask_id;
    a.pv = pv;
    a.pi = pi;
    const int grid = rx_grid(w, M);
    a.parts = grid;
    *parts = a.parts;
    return run_rx<1>(w, a, M, grid, st);
}

hipError_t gemm_mfma(const DevMatrix &w, const float *X, int ldx, int M, float *Y, int ldy, const float *bias,
                     bool relu, const float *R, int ldr, hipStream_t st, float *ws, size_t ws_bytes) {
    if (M <= 0) return hipSuccess;
    if (!gemm_mfma_supported(w) || ldx % 4 || reinterpret_cast<uintptr_t>(X) % 16) return hipErrorInvalidValue;
    if (gemm_rx_supported(w, M) && w.N >= kRxMinRows) {
        RxArgs r = rx_args(w, X, ldx, M);
        r.y = Y;
        r.ldy = ldy;
        r.bias = bias;
        r.R = R;
        r.ldr = ldr;
        r.relu = relu ? 1 : 0;
        return run_rx<0>(w, r, M, rx_grid(w, M), st);
    }
    MfmaArgs a{};
    a.w = wptr_of(w);
    a.x = X;
    a.ldx = ldx;
    a.M = M;
    a.y = Y;
    a.ldy = ldy;
    a.bias = bias;
    a.R = R;
    a.ldr = ldr;
    a.relu = relu ? 1 : 0;
    const int ks = ws ? split_k(w, M, ws_bytes) : 1;
    a.part = ks > 1 ? ws : nullptr;
    hipError_t e;
    switch (w.type) {
    case GGML_Q4_K: e = launch<GGML_Q4_K>(a, M, ks, st); break;
    case GGML_Q5_K: e = launch<GGML_Q5_K>(a, M, ks, st); break;
    case GGML_Q6_K: e = launch<GGML_Q6_K>(a, M, ks, st); break;
    case GGML_Q8_0: e = launch<GGML_Q8_0>(a, M, ks, st); break;
    case GGML_F16: e = launch<GGML_F16>(a, M, ks, st); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess || ks == 1) return e;
    const size_t mn = size_t(M) * w.N;
    hipLaunchKernelGGL(k_splitk_reduce, dim3(unsigned((mn + 255) / 256)), dim3(256), 0, st, ws, ks, M, w.N, bias, R,
                       ldr, relu ? 1 : 0, Y, ldy);
    return hipGetLastError();
}


namespace {
// Runs the tile kernel with K split over workgroups into ws; returns the split
// count (1: not split, nothing launched).
int launch_split(const DevMatrix &w, const float *X, int ldx, int M, hipStream_t st, float *ws, size_t ws_bytes,
                 hipError_t *err) {
    *err = hipSuccess;
    if (!ws || !gemm_mfma_supported(w) || ldx % 4 || reinterpret_cast<uintptr_t>(X) % 16) return 1;
    if (gemm_rx_supported(w, M) && w.N >= kRxMinRows) return 1;
    const int ks = split_k(w, M, ws_bytes);
    if (ks <= 1) return 1;
    MfmaArgs a{};
    a.w = wptr_of(w);
    a.x = X;
    a.ldx = ldx;
    a.M = M;
    a.part = ws;
    switch (w.type) {
    case GGML_Q4_K: *err = launch<GGML_Q4_K>(a, M, ks, st); break;
    case GGML_Q5_K: *err = launch<GGML_Q5_K>(a, M, ks, st); break;
    case GGML_Q6_K: *err = launch<GGML_Q6_K>(a, M, ks, st); break;
    case GGML_Q8_0: *err = launch<GGML_Q8_0>(a, M, ks, st); break;
    case GGML_F16: *err = launch<GGML_F16>(a, M, ks, st); break;
    default: return 1;
    }
    return ks;
}
}  // namespace

hipError_t gemm_residual_ln(const DevMatrix &w, const float *X, int ldx, int M, const float *bias, float *x,
                            const float *g, const float *b, float eps, float *h, hipStream_t st, float *ws,
                            size_t ws_bytes) {
    if (M <= 0) return hipSuccess;
    if (w.N > 4096 || w.N % 4) return hipErrorInvalidValue;
    hipError_t e;
    const int ks = launch_split(w, X, ldx, M, st, ws, ws_bytes, &e);
    if (e != hipSuccess) return e;
    if (ks > 1) {
        hipLaunchKernelGGL(k_splitk_residual_ln, dim3(M), dim3(256), 0, st, ws, ks, M, w.N, bias, x, g, b, eps, h);
        return hipGetLastError();
    }
    // x = x + X W^T + bias in place (R = Y = x), then the LayerNorm
    e = gemm(w, X, ldx, M, x, w.N, bias, false, x, w.N, st, ws, ws_bytes);
    if (e != hipSuccess) return e;
    return layernorm(x, M, w.N, g, b, eps, h, st);
}

namespace {
template <typename KT>
hipError_t gemm_qkv_t(const DevMatrix &w, const float *X, int ldx, int M, const float *bias, int H, int hd, int slots,
                      const uint32_t *step, float *q, KT *kc, KT *vc, float *qkv_tmp, hipStream_t st, float *ws,
                      size_t ws_bytes) {
    if (M <= 0) return hipSuccess;
    const int d = H * hd;
    if (w.N != 3 * d) return hipErrorInvalidValue;
    hipError_t e;
    const int ks = launch_split(w, X, ldx, M, st, ws, ws_bytes, &e);
    if (e != hipSuccess) return e;
    if (ks > 1) {
        const size_t n = size_t(M) * w.N;
        hipLaunchKernelGGL(k_splitk_qkv<KT>, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, ws, ks, M, d, bias, H,
                           hd, slots, step, q, kc, vc);
        return hipGetLastError();
    }
    e = gemm(w, X, ldx, M, qkv_tmp, w.N, bias, false, nullptr, 0, st, ws, ws_bytes);
    if (e != hipSuccess) return e;
    return qkv_split(qkv_tmp, M, H, hd, slots, step, q, kc, vc, st);
}
}  // namespace

hipError_t gemm_qkv(const DevMatrix &w, const float *X, int ldx, int M, const float *bias, int H, int hd, int slots,
                    const uint32_t *step, float *q, __half *kc, __half *vc, float *qkv_tmp, hipStream_t st, float *ws,
                    size_t ws_bytes) {
    return gemm_qkv_t(w, X, ldx, M, bias, H, hd, slots, step, q, kc, vc, qkv_tmp, st, ws, ws_bytes);
}

hipError_t gemm_qkv(const DevMatrix &w, const float *X, int ldx, int M, const float *bias, int H, int hd, int slots,
                    const uint32_t *step, float *q, float *kc, float *vc, float *qkv_tmp, hipStream_t st, float *ws,
                    size_t ws_bytes) {
    return gemm_qkv_t(w, X, ldx, M, bias, H, hd, slots, step, q, kc, vc, qkv_tmp, st, ws, ws_bytes);
}

}  // namespace mlg
