// Dequant GEMM for many rows (encoder prefill, batched decode when the
// register-resident GEMV does not apply): Y = X W^T + bias (+ R) (relu).
// SIMT f32: a 64(n) x 32(m) output tile per 256-thread workgroup, K in steps of
// 64; the weight tile is dequantized into LDS once per step and shared by all
// 32 rows of X.
#include "dequant.hpp"
#include "kernels.hpp"

namespace mlg {

namespace {

constexpr int BN = 64, BM = 32, BK = 64;

template <int T>
__global__ __launch_bounds__(256) void k_gemm(const uint8_t *__restrict__ q, const uint8_t *__restrict__ s,
                                              const uint8_t *__restrict__ dp, int N, int K,
                                              const float *__restrict__ X, int ldx, int M, float *Y, int ldy,
                                              const float *__restrict__ bias, int relu, const float *R, int ldr) {
    __shared__ float Ws[BK][BN + 1];
    __shared__ float Xs[BK][BM + 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    float acc[2][4] = {};
    for (int k0 = 0; k0 < K; k0 += BK) {
        // weights: thread -> (row n0 + tid/4, 16 values at k0 + 16*(tid%4))
        {
            const int nr = tid >> 2, kk = (tid & 3) * 16;
            float w[16];
            const int n = n0 + nr;
            if (n < N && k0 + kk < K) {
                dequant16<T>(q, s, dp, K, n, k0 + kk, w);
            } else {
#pragma unroll
                for (int e = 0; e < 16; ++e) w[e] = 0.f;
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) Ws[kk + e][nr] = w[e];
        }
        // activations: 32 rows x 64 k -> 8 values per thread
        {
            const int mr = tid >> 3, kk = (tid & 7) * 8;
            const int m = m0 + mr;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int k = k0 + kk + e;
                Xs[kk + e][mr] = (m < M && k < K) ? X[size_t(m) * ldx + k] : 0.f;
            }
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < BK; ++k) {
            const float a0 = Xs[k][ty * 2], a1 = Xs[k][ty * 2 + 1];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float w = Ws[k][tx * 4 + j];
                acc[0][j] = fmaf(a0, w, acc[0][j]);
                acc[1][j] = fmaf(a1, w, acc[1][j]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int m = m0 + ty * 2 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n >= N) continue;
            float v = acc[i][j];
            if (bias) v += bias[n];
            if (R) v = R[size_t(m) * ldr + n] + v;
            if (relu) v = fmaxf(v, 0.f);
            Y[size_t(m) * ldy + n] = v;
        }
    }
}

template <int T>
hipError_t launch(const DevMatrix &w, const float *X, int ldx, int M, float *Y, int ldy, const float *bias, bool relu,
                  const float *R, int ldr, hipStream_t st) {
    dim3 grid((w.N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL(k_gemm<T>, grid, dim3(256), 0, st, w.q, w.s, w.d, w.N, w.K, X, ldx, M, Y, ldy, bias,
                       relu ? 1 : 0, R, ldr);
    return hipGetLastError();
}

}  // namespace

hipError_t gemm_simt(const DevMatrix &w, const float *X, int ldx, int M, float *Y, int ldy, const float *bias,
                     bool relu, const float *R, int ldr, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    if (w.K % 16) return hipErrorInvalidValue;
    MLG_DISPATCH_TYPE(w.type, launch, w, X, ldx, M, Y, ldy, bias, relu, R, ldr, st)
}

hipError_t gemm(const DevMatrix &w, const float *X, int ldx, int M, float *Y, int ldy, const float *bias, bool relu,
                const float *R, int ldr, hipStream_t st, float *ws, size_t ws_bytes) {
    if (gemm_mfma_supported(w) && ldx % 4 == 0 && reinterpret_cast<uintptr_t>(X) % 16 == 0)
        return gemm_mfma(w, X, ldx, M, Y, ldy, bias, relu, R, ldr, st, ws, ws_bytes);
    return gemm_simt(w, X, ldx, M, Y, ldy, bias, relu, R, ldr, st);
}

}  // namespace mlg
