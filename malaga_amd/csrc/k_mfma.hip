// Dequant GEMM on the MFMA units (src/model.rs:463-477 encoder prefill, and the
// projections of decode batches too large for the register GEMV):
//   Y[m][n] = sum_k X[m][k] W[n][k] + bias[n] (+ R[m][n]) (relu)
//
// Exactness: the integer quants (q4_K / q5_K nibbles, q6_K 6-bit values - 32,
// q8_0 int8) are exact in f16, so the MFMA multiplies them by X, which is split
// into two f16 terms x = hi + lo (|x - hi - lo| <= 2^-22 |x|), with f32
// accumulation; block scales and k-quant mins are applied per sub-block in f32:
//   sum_k w_k x_k = d sc * sum_k q_k x_k - dmin m * sum_k x_k.
//
// Tiling: a workgroup (4 waves) owns 64 rows of W (16 per wave) and BM rows of X.
// K is consumed in steps of 256 (one k-quant super-block): the X step is staged
// in LDS as hi/lo f16 plus per-16 sums, while the next step's X and W are in
// flight in registers.  Each wave keeps its W rows in registers in the MFMA
// B-operand layout (lane l: row l % 16, k-group l / 16) and reads A (X) from LDS.
// f16 MFMA operand conversion of quant bytes uses v_perm (byte -> 0x64xx = 1024 +
// byte) and one packed f16 subtraction.
#include "device.hpp"
#include "gemv_core.hpp"
#include "kernels.hpp"

#include <algorithm>

namespace mlg {

namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kStep = 256;        // K per staging step
constexpr int kXS = kStep + 8;    // LDS row stride of the staged X (halves)
constexpr int kTileN = 64;        // W rows per workgroup

struct MfmaArgs {
    WPtr w;
    const float *x;
    int ldx, M;
    float *y;
    int ldy;
    const float *bias, *R;
    int ldr, relu;
    float *part;  // split K: raw sums [gridDim.z][M][N], epilogue in k_splitk_reduce
};

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

// q4_K: 8 sub-blocks of 32; lane k-group kq reads bytes qs[32 g + 8 kq, +8) of the
// 4 byte groups g (low nibbles: sub-block 2g, high nibbles: 2g + 1).
template <>
struct MW<GGML_Q4_K> {
    static constexpr int SLICES = 8, SK = 32;
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
};

// q5_K: as q4_K plus the fifth bit of sub-block s in bit s of qh[l] (l < 32).
template <>
struct MW<GGML_Q5_K> {
    static constexpr int SLICES = 8, SK = 32;
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
};

// q6_K: 16 groups of 16 with an int8 scale each (one 16x16x16 MFMA per group).
// Group G = 8 n + 2 t + h holds values 128 n + 32 t + 16 h + j (j < 16): low 4 bits
// from ql[64 n + 32 (t & 1) + 16 h + j] (nibble t >> 1), high 2 bits from
// qh[32 n + 16 h + j] bits 2t..2t+1.  Lane k-group kq takes j = 4 kq .. 4 kq + 3.
template <>
struct MW<GGML_Q6_K> {
    static constexpr int SLICES = 16, SK = 16;
    struct Regs {
        uint32_t qa[4], qb[4], qh[4];  // [2 n + h]
        uint4 sc;
        uint32_t d;
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
};

// q8_0: 8 blocks of 32 per step, int8 values (q ^ 0x80 = q + 128 as a byte).
template <>
struct MW<GGML_Q8_0> {
    static constexpr int SLICES = 8, SK = 32;
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

template <int T, int BM>
__global__ __launch_bounds__(256) void k_mfma(MfmaArgs a) {
    using W = MW<T>;
    constexpr int MT = BM / 16;     // 16-row tiles of X
    constexpr int FPT = BM;         // X values staged per thread and step (BM * 256 / 256)
    constexpr int TPR = 256 / BM;   // threads per X row
    __shared__ _Float16 xh[BM * kXS], xl[BM * kXS];
    __shared__ float xsum[16 * BM];  // [16-slice][m]
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int kq = lane >> 4, ln = lane & 15;
    const int n0 = blockIdx.x * kTileN + 16 * w;
    const int row = min(n0 + ln, a.w.N - 1);
    const int m0 = blockIdx.y * BM;
    // K steps [kb0, kb1) of this split
    const int nsteps = a.w.K / kStep, ks = gridDim.z;
    const int kb0 = int(blockIdx.z) * nsteps / ks, kb1 = (int(blockIdx.z) + 1) * nsteps / ks;

    // X staging: thread t owns row m0 + t / TPR, values [(t % TPR) FPT, +FPT) of the step
    const int xm = t / TPR, xk = (t % TPR) * FPT;
    const bool xrow_ok = m0 + xm < a.M;
    const float *xsrc = a.x + size_t(xrow_ok ? m0 + xm : 0) * a.ldx + xk;
    float4 xr[FPT / 4];
    auto load_x = [&](int kb) {
#pragma unroll
        for (int i = 0; i < FPT / 4; ++i)
            xr[i] = xrow_ok ? *reinterpret_cast<const float4 *>(xsrc + size_t(kb) * kStep + 4 * i)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto stage_x = [&] {
#pragma unroll
        for (int i = 0; i < FPT / 4; ++i) {
            const float v[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
            _Float16 hv[4], lv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                hv[e] = _Float16(v[e]);
                lv[e] = _Float16(v[e] - float(hv[e]));
            }
            *reinterpret_cast<h4_t *>(xh + xm * kXS + xk + 4 * i) = h4_t{hv[0], hv[1], hv[2], hv[3]};
            *reinterpret_cast<h4_t *>(xl + xm * kXS + xk + 4 * i) = h4_t{lv[0], lv[1], lv[2], lv[3]};
        }
#pragma unroll
        for (int j = 0; j < FPT / 16; ++j) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) s += (xr[4 * j + i].x + xr[4 * j + i].y) + (xr[4 * j + i].z + xr[4 * j + i].w);
            xsum[((xk >> 4) + j) * BM + xm] = s;
        }
    };

    f4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f4_t{0.f, 0.f, 0.f, 0.f};

    typename W::Regs cur, nxt;
    W::load(a.w, row, kb0, kq, cur);
    load_x(kb0);
    for (int kb = kb0; kb < kb1; ++kb) {
        if (kb != kb0) lds_barrier();  // the previous step's reads of xh / xl / xsum are done
        stage_x();
        lds_barrier();
        if (kb + 1 < kb1) {
            W::load(a.w, row, kb + 1, kq, nxt);
            load_x(kb + 1);
        }
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
    float v = part[i];
    for (int z = 1; z < ks; ++z) v += part[size_t(z) * mn + i];
    if (bias) v += bias[n];
    if (R) v += R[size_t(m) * ldr + n];
    if (relu) v = fmaxf(v, 0.f);
    y[size_t(m) * ldy + n] = v;
}

template <int T>
hipError_t launch(const MfmaArgs &a, int M, int ks, hipStream_t st) {
    const int gx = (a.w.N + kTileN - 1) / kTileN;
    if (M <= 16) {
        hipLaunchKernelGGL((k_mfma<T, 16>), dim3(gx, (M + 15) / 16, ks), dim3(256), 0, st, a);
    } else if (M <= 32) {
        hipLaunchKernelGGL((k_mfma<T, 32>), dim3(gx, 1, ks), dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL((k_mfma<T, 64>), dim3(gx, (M + 63) / 64, ks), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

// K splits that bring the grid to about one workgroup per CU, within the workspace
int split_k(const DevMatrix &w, int M, size_t ws_bytes) {
    const int gx = (w.N + kTileN - 1) / kTileN, bm = M <= 16 ? 16 : M <= 32 ? 32 : 64;
    const int base = gx * ((M + bm - 1) / bm), nsteps = w.K / kStep;
    int ks = base >= 256 ? 1 : std::min(nsteps, (256 + base - 1) / base);
    while (ks > 1 && size_t(ks) * M * w.N * sizeof(float) > ws_bytes) --ks;
    return ks;
}

}  // namespace

bool gemm_mfma_supported(const DevMatrix &w) {
    const bool type_ok = w.type == GGML_Q4_K || w.type == GGML_Q5_K || w.type == GGML_Q6_K ||
                         w.type == GGML_Q8_0 || w.type == GGML_F16;
    return type_ok && w.K % kStep == 0 && w.N > 0;
}

hipError_t gemm_mfma(const DevMatrix &w, const float *X, int ldx, int M, float *Y, int ldy, const float *bias,
                     bool relu, const float *R, int ldr, hipStream_t st, float *ws, size_t ws_bytes) {
    if (M <= 0) return hipSuccess;
    if (!gemm_mfma_supported(w) || ldx % 4 || reinterpret_cast<uintptr_t>(X) % 16) return hipErrorInvalidValue;
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

}  // namespace mlg
