// Device-side helpers shared by the HIP kernels (gfx950, wave64).
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlg {

constexpr int kWave = 64;

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits16 & 0xffffu)));
}

// byte b (0..3) of a dword as float: one v_cvt_f32_ubyteN each
__device__ __forceinline__ float ub0(uint32_t v) {
    float r;
    asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    return r;
}
__device__ __forceinline__ float ub1(uint32_t v) {
    float r;
    asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    return r;
}
__device__ __forceinline__ float ub2(uint32_t v) {
    float r;
    asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    return r;
}
__device__ __forceinline__ float ub3(uint32_t v) {
    float r;
    asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// 4 products of the bytes of v with x[0..3], accumulated into acc
__device__ __forceinline__ float dot4u8(uint32_t v, const float *x, float acc) {
    acc = fmaf(ub0(v), x[0], acc);
    acc = fmaf(ub1(v), x[1], acc);
    acc = fmaf(ub2(v), x[2], acc);
    acc = fmaf(ub3(v), x[3], acc);
    return acc;
}

// Workgroup barrier that waits only for this wave's LDS traffic (lgkmcnt(0)), not
// for outstanding global loads, so prefetched weights stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // vmcnt: no wait, expcnt: no wait, lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int W>
__device__ __forceinline__ float group_sum(float v) {
    // sum within aligned groups of W lanes (W power of two, <= 64)
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<kWave>(v); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// (value, index) argmax step: larger value wins, ties go to the lower index.
__device__ __forceinline__ void argmax_merge(float &v, uint32_t &i, float ov, uint32_t oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__device__ __forceinline__ void wave_argmax(float &v, uint32_t &i) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const uint32_t oi = __shfl_xor(i, o, kWave);
        argmax_merge(v, i, ov, oi);
    }
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024).  `sh` holds >= 16 floats.
__device__ __forceinline__ float block_sum(float v, float *sh) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) sh[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int k = 0; k < nw; ++k) t += sh[k];
    return t;
}

__device__ __forceinline__ float block_max(float v, float *sh) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_max(v);
    __syncthreads();
    if (lane == 0) sh[w] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int k = 0; k < nw; ++k) t = fmaxf(t, sh[k]);
    return t;
}

// 6-bit (scale, min) pair j of a Q4_K / Q5_K block; s0..s2 are the 12 scale bytes.
__device__ __forceinline__ void k4_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2, float &sc, float &m) {
    const uint32_t w[3] = {s0, s1, s2};
    auto byte = [&](int k) { return (w[k >> 2] >> (8 * (k & 3))) & 0xffu; };
    uint32_t a, b;
    if (j < 4) {
        a = byte(j) & 63;
        b = byte(j + 4) & 63;
    } else {
        a = (byte(j + 4) & 0xf) | ((byte(j - 4) >> 6) << 4);
        b = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
    sc = float(a);
    m = float(b);
}

}  // namespace mlg
