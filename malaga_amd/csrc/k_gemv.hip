// Stand-alone dequant-GEMV kernels (batch 1..4): y = x W^T (+ bias) (relu), and
// the LM-head variant whose epilogue keeps a per-workgroup argmax instead of
// storing the logits.  The streaming core is gemv_core.hpp.
#include <map>
#include <mutex>
#include <tuple>

#include "gemv_core.hpp"
#include "kernels.hpp"

namespace mlg {

namespace {

struct GemvArgs {
    WPtr w;
    GemvGeom g;
    const float *x;
    int ldx, nb;
    float *y;
    int ldy;
    const float *bias;
    int relu;
    float *pv;  // argmax partials [nb][gridDim.x]
    uint32_t *pi;
    int mask_id;
    int nt_from;  // LM head: first row loaded non-temporally
    // LM head: x = LayerNorm(ln_x + ln_y) (ln_g, ln_b, ln_eps) computed by every
    // workgroup (workgroup 0 also stores it to ln_h); a.x is unused then
    const float *ln_x, *ln_y, *ln_g, *ln_b;
    float ln_eps;
    float *ln_h;
};

template <int B>
struct StoreEpi {
    const GemvArgs &a;
    __device__ void operator()(int row, int bi, float v) const {
        if (bi >= a.nb) return;
        if (a.relu) v = fmaxf(v, 0.f);
        a.y[size_t(bi) * a.ldy + row] = v;
    }
};

template <int B>
struct ArgmaxEpi {
    const GemvArgs &a;
    float best[B];
    uint32_t idx[B];
    __device__ void operator()(int row, int bi, float v) {
        if (row != a.mask_id) argmax_merge(best[bi], idx[bi], v, uint32_t(row));
    }
};

// MODE 0: store (small, latency-bound matrices, f32 x); MODE 2: store, large matrices
// (limb x, one resident round of workgroups); MODE 1: LM head with argmax partials,
// mostly non-temporal weights.  One row group per wave step (G = 1) in all three:
// fewer registers, more waves per SIMD (measured faster than G = 2 for the large ones).
// LM head: three steps of weights requested per wave (two for the other GEMVs)
constexpr int kLmHeadDepth = 3;

template <int T, int MODE>
constexpr bool kGemvLimbs = MODE != 0 && kLimbX<T>;  // large matrices: limb x (gemv_core.hpp)

// LM: a.w.q is the lane-major quant copy of a q6_K head (DevMatrix::lm)
// L2 > 0: lanes per row group = 2^L2 at compile time (a.g.lpr_log2 == L2)
template <int T, int B, int CPL, int MODE, bool LM, int L2 = 0>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
    extern __shared__ uint32_t xlds[];  // limbs of x
    const int lane = threadIdx.x & 63;
    const int cl = lane & ((1 << (L2 > 0 ? L2 : a.g.lpr_log2)) - 1);
    XRep<T, B, kGemvLimbs<T, MODE>> xr[CPL];
    auto load_x = [&] {
        if constexpr (kGemvLimbs<T, MODE>) {
            if (MODE == 1 && a.ln_x) {
                // h = LayerNorm(ln_x + ln_y) (biased variance, f64 statistics), each row
                // spread over the workgroup's 256 threads, into LDS after the limbs
                __shared__ double red[8];
                const int K = a.w.K;
                float *hs = reinterpret_cast<float *>(xlds) + xq_lds_bytes<T>(K, a.nb) / 4;
                for (int bi = 0; bi < a.nb; ++bi) {  // workgroup-uniform
                    const float4 *xr = reinterpret_cast<const float4 *>(a.ln_x + size_t(bi) * K);
                    const float4 *yr = reinterpret_cast<const float4 *>(a.ln_y + size_t(bi) * K);
                    auto form = [&](int f) {
                        float4 v = xr[f];
                        add4(v, yr[f]);
                        return v;
                    };
                    workgroup_row_layernorm<kWaveLnMaxD / 1024>(K, form, NoKeep{}, a.ln_g, a.ln_b, a.ln_eps,
                                                                hs + size_t(bi) * K, red);
                }
                __syncthreads();
                if (blockIdx.x == 0 && a.ln_h)
                    for (int i = threadIdx.x; i < a.nb * K; i += blockDim.x) a.ln_h[i] = hs[i];
                stage_limbs<T>(hs, K, a.nb, K, xlds);
            } else {
                stage_limbs<T>(a.x, a.ldx, a.nb, a.w.K, xlds);
            }
            lds_barrier();
            gemv_load_xq<T, B, CPL>(xlds, a.w.K, a.nb, a.g, cl, xr);
        } else {
            gemv_load_x<T, B, CPL>(a.x, a.ldx, a.nb, a.g, cl, xr);
        }
    };
    // a scalar: the per-step branches on it stay uniform (no divergent load paths)
    const int gwave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6)), nwaves = gridDim.x * 4;
    if constexpr (MODE == 0) {
        StoreEpi<B> epi{a};
        gemv_rows<T, B, CPL, false, 1, LM>(a.w, a.g, xr, gwave, nwaves, NoPre{}, load_x, epi, a.bias);
    } else if constexpr (MODE == 2) {
        StoreEpi<B> epi{a};
        gemv_rows<T, B, CPL, false, 1, LM, L2>(a.w, a.g, xr, gwave, nwaves, NoPre{}, load_x, epi, a.bias);
    } else {  // the LM head: weights streamed once per step
        ArgmaxEpi<B> epi{a, {}, {}};
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            epi.best[bi] = -INFINITY;
            epi.idx[bi] = 0xffffffffu;
        }
        // rows >= nt_from non-temporal: the 215 MB stream then evicts less of the layer
        // weights from the MALL between steps (measured: -20 us per 600M step)
        gemv_rows<T, B, CPL, true, 1, LM, L2, kLmHeadDepth>(a.w, a.g, xr, gwave, nwaves, NoPre{}, load_x, epi,
                                                            a.bias, a.nt_from);
        __shared__ float sv[4][B];
        __shared__ uint32_t si[4][B];
        const int wv = threadIdx.x >> 6;
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            wave_argmax(epi.best[bi], epi.idx[bi]);
            if (lane == 0) {
                sv[wv][bi] = epi.best[bi];
                si[wv][bi] = epi.idx[bi];
            }
        }
        __syncthreads();
        if (int(threadIdx.x) < B && int(threadIdx.x) < a.nb) {
            const int bi = threadIdx.x;
            float v = sv[0][bi];
            uint32_t i = si[0][bi];
            for (int k = 1; k < 4; ++k) argmax_merge(v, i, sv[k][bi], si[k][bi]);
            a.pv[size_t(bi) * gridDim.x + blockIdx.x] = v;
            a.pi[size_t(bi) * gridDim.x + blockIdx.x] = i;
        }
    }
}

// Workgroups of one launch that are resident on the device at once (CUs x blocks per
// CU at this kernel's occupancy with `lds` dynamic LDS bytes), or 0 if the runtime
// cannot say.  Remembered per (kernel, device, LDS bytes).
inline int resident_grid(const void *kernel, int lds) {
    static std::mutex mu;
    static std::map<std::tuple<const void *, int, int>, int> known;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    const auto key = std::make_tuple(kernel, dev, lds);
    std::lock_guard<std::mutex> lk(mu);
    auto it = known.find(key);
    if (it != known.end()) return it->second;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, size_t(lds)) != hipSuccess)
        return 0;
    return known[key] = cus * per_cu;
}

// Static LDS of k_gemv: the argmax epilogue's per-wave (value, index) pairs and the
// folded LayerNorm's wave sums.
constexpr int kGemvStaticLds = 4 * 4 * (sizeof(float) + sizeof(uint32_t)) + 8 * sizeof(double);

// grid: in, the workgroups that cover the rows; out, the workgroups launched.  The
// large-matrix modes launch at most one resident round (each wave then streams its
// rows to the end): with more workgroups than fit at once, the last round runs part
// empty (measured on the 600M LM head: 2048 workgroups 46.2 us, 1536 45.1 us, one
// round of 768 42.5 us).
// launch = false: only the grid is set (the partial count gemv_argmax_parts reports).
template <int T, int B, int CPL, int MODE, bool LM, int L2 = 0>
hipError_t launch_t(const GemvArgs &a, int &grid, hipStream_t st, bool launch) {
    if constexpr (GTraits<T>::XW * B * CPL > kGemvMaxXRegs) {
        return hipErrorInvalidValue;
    } else {
        const int lds = (kGemvLimbs<T, MODE> ? xq_lds_bytes<T>(a.w.K, a.nb) : 0) +
                        (MODE == 1 && a.ln_x ? a.nb * a.w.K * int(sizeof(float)) : 0);
        if (lds + kGemvStaticLds > 65536) return hipErrorInvalidValue;
        if constexpr (MODE != 0) {
            // the occupancy of this launch's LDS bytes (limbs of nb rows, the folded
            // LayerNorm's rows)
            const int resident = resident_grid(reinterpret_cast<const void *>(&k_gemv<T, B, CPL, MODE, LM, L2>), lds);
            if (resident > 0 && grid > resident) grid = resident;
        }
        if (!launch) return hipSuccess;
        hipLaunchKernelGGL((k_gemv<T, B, CPL, MODE, LM, L2>), dim3(grid), dim3(256), lds, st, a);
        return hipGetLastError();
    }
}

template <int T, int MODE, bool LM = false>
hipError_t dispatch_bc(const GemvArgs &a, int B, int cpl, int &grid, hipStream_t st, bool launch) {
    if constexpr (MODE != 0) {  // batch-1 large GEMVs of K = 1024 (16 or 32 lanes per row) and 2048
        if (B == 1 && cpl == 1 && a.g.lpr_log2 == 4) return launch_t<T, 1, 1, MODE, LM, 4>(a, grid, st, launch);
        if (B == 1 && cpl == 1 && a.g.lpr_log2 == 5) return launch_t<T, 1, 1, MODE, LM, 5>(a, grid, st, launch);
    }
#define MLG_CASE(BB, CC) \
    if (B == BB && cpl == CC) return launch_t<T, BB, CC, MODE, LM>(a, grid, st, launch);
    MLG_CASE(1, 1) MLG_CASE(1, 2) MLG_CASE(1, 4)
    MLG_CASE(2, 1) MLG_CASE(2, 2) MLG_CASE(2, 4)
    MLG_CASE(4, 1) MLG_CASE(4, 2) MLG_CASE(4, 4)
#undef MLG_CASE
    return hipErrorInvalidValue;
}

// lm: lane-major quants of a q6_K head (the large-matrix modes only)
template <int MODE>
hipError_t dispatch(uint32_t type, const GemvArgs &a, int B, int cpl, int &grid, hipStream_t st,
                    const uint8_t *lm = nullptr, bool launch = true) {
    switch (type) {
    case GGML_Q4_K: return dispatch_bc<GGML_Q4_K, MODE>(a, B, cpl, grid, st, launch);
    case GGML_Q5_K: return dispatch_bc<GGML_Q5_K, MODE>(a, B, cpl, grid, st, launch);
    case GGML_Q6_K:
        if constexpr (MODE != 0) {
            if (lm) {
                GemvArgs b = a;
                b.w.q = lm;
                return dispatch_bc<GGML_Q6_K, MODE, true>(b, B, cpl, grid, st, launch);
            }
        }
        return dispatch_bc<GGML_Q6_K, MODE>(a, B, cpl, grid, st, launch);
    case GGML_Q8_0: return dispatch_bc<GGML_Q8_0, MODE>(a, B, cpl, grid, st, launch);
    case GGML_F16: return dispatch_bc<GGML_F16, MODE>(a, B, cpl, grid, st, launch);
    case GGML_F32: return dispatch_bc<GGML_F32, MODE>(a, B, cpl, grid, st, launch);
    default: return hipErrorInvalidValue;
    }
}

GemvArgs make_args(const DevMatrix &w, const GemvGeom &g, const float *x, int ldx, int b) {
    GemvArgs a{};
    a.w = wptr_of(w);
    a.g = g;
    a.x = x;
    a.ldx = ldx;
    a.nb = b;
    a.mask_id = -1;
    return a;
}

constexpr int kGemvSmallRows = 65536;

// An LM head of at most kLmHeadCachedBytes (a 37k-row shortlist is 31 MB) is read with
// cached loads, so that it stays in the 256 MB MALL from step to step; a larger one is
// streamed non-temporally, so that its pass evicts less of the layer weights (112 MB
// for 600M q4_k_m) between steps.  Measured on the 600M head (215 MB): an all
// non-temporal stream 38.1 us against 38.7 us with its first 32 MB cached, and on
// batch-1 decode a cached prefix of 0, 16 or 32 MB within noise (64 MB 0.15 ms per
// sentence slower, 128 MB 0.6 ms).
constexpr size_t kLmHeadCachedBytes = 32000000;

}  // namespace

int gemv_grid(const DevMatrix &w, int G) {
    GemvGeom g;
    int cpl;
    if (!gemv_geometry(w, &g, &cpl)) return 0;
    const int rpw = 64 >> g.lpr_log2;
    const int groups = (w.N + rpw - 1) / rpw;
    // G row groups per wave and step; capped at 2048 workgroups (the large-matrix modes
    // then launch at most one resident round: launch_t)
    const int waves = (groups + G - 1) / G;
    const int grid = (waves + 3) / 4;
    return grid < 1 ? 1 : (grid > 2048 ? 2048 : grid);
}

int gemv_max_batch(const DevMatrix &w) {
    GemvGeom g;
    int cpl;
    if (!gemv_geometry(w, &g, &cpl)) return 0;
    const int xw = gemv_xw(w.type);
    int best = 0;
    for (int b : {1, 2, 4})
        if (xw * b * cpl <= kGemvMaxXRegs) best = b;
    return best;
}

hipError_t gemv(const DevMatrix &w, const float *x, int ldx, int b, float *y, int ldy, const float *bias, bool relu,
                hipStream_t st) {
    GemvGeom g;
    int cpl;
    if (b < 1 || b > gemv_max_batch(w) || !gemv_geometry(w, &g, &cpl) || ldx % 4 ||
        reinterpret_cast<uintptr_t>(x) % 16)
        return hipErrorInvalidValue;
    GemvArgs a = make_args(w, g, x, ldx, b);
    a.y = y;
    a.ldy = ldy;
    a.bias = bias;
    a.relu = relu ? 1 : 0;
    if (w.N <= kGemvSmallRows) {
        int grid = gemv_grid(w, 1);
        return dispatch<0>(w.type, a, gemv_round_b(b), cpl, grid, st);
    }
    int grid = gemv_grid(w, 1);
    return dispatch<2>(w.type, a, gemv_round_b(b), cpl, grid, st, w.lm);
}

int gemv_argmax_parts(const DevMatrix &w, int b) {
    GemvGeom g;
    int cpl;
    if (b < 1 || b > gemv_max_batch(w) || !gemv_geometry(w, &g, &cpl)) return gemv_grid(w, 1);
    GemvArgs a = make_args(w, g, nullptr, 0, b);
    int grid = gemv_grid(w, 1);
    (void)dispatch<1>(w.type, a, gemv_round_b(b), cpl, grid, nullptr, w.lm, false);  // the grid only: no launch
    return grid;
}

hipError_t gemv_argmax(const DevMatrix &w, const float *x, int ldx, int b, int mask_id, float *pv, uint32_t *pi,
                       int *parts, hipStream_t st, const GemvLn *ln) {
    GemvGeom g;
    int cpl;
    if (b < 1 || b > gemv_max_batch(w) || !gemv_geometry(w, &g, &cpl) || ldx % 4 ||
        reinterpret_cast<uintptr_t>(x) % 16)
        return hipErrorInvalidValue;
    GemvArgs a = make_args(w, g, x, ldx, b);
    a.pv = pv;
    a.pi = pi;
    a.mask_id = mask_id;
    if (ln) {
        if (!(w.type == GGML_Q4_K || w.type == GGML_Q5_K || w.type == GGML_Q6_K || w.type == GGML_Q8_0) ||
            w.K > kWaveLnMaxD || w.K % 4)
            return hipErrorInvalidValue;
        a.ln_x = ln->x;
        a.ln_y = ln->y;
        a.ln_g = ln->g;
        a.ln_b = ln->b;
        a.ln_eps = ln->eps;
        a.ln_h = ln->h;
    }
    int grid = gemv_grid(w, 1);
    a.nt_from = w.bytes <= kLmHeadCachedBytes ? w.N : 0;  // first row streamed non-temporally
    const hipError_t e = dispatch<1>(w.type, a, gemv_round_b(b), cpl, grid, st, w.lm);
    *parts = grid;  // the workgroups launched, = gemv_argmax_parts(w, b)
    return e;
}

}  // namespace mlg
