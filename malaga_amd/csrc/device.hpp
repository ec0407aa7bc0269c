// Device-side helpers shared by the HIP kernels (gfx950, wave64).
#pragma once
#include <type_traits>
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

// Cross-lane moves with DPP (no LDS round trip).  Every helper below must be
// called with all 64 lanes active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
    return uint32_t(__builtin_amdgcn_mov_dpp(int(v), CTRL, 0xf, 0xf, true));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- lane 7 - i within 8
constexpr int kDppMirror = 0x140;      // lane i <- lane 15 - i within 16

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Reduction within aligned groups of 2^log2w lanes (log2w <= 6, wave-uniform);
// every lane of a group receives the same, bitwise identical result.  Each step
// combines the lane with one in the other half of its current group, so the
// combining order does not depend on the lane.
template <class Op>
__device__ __forceinline__ float group_reduce(float v, int log2w, Op op) {
    if (log2w >= 1) v = op(v, dpp_mov<kDppXor1>(v));
    if (log2w >= 2) v = op(v, dpp_mov<kDppXor2>(v));
    if (log2w >= 3) v = op(v, dpp_mov<kDppHalfMirror>(v));
    if (log2w >= 4) v = op(v, dpp_mov<kDppMirror>(v));
    if (log2w >= 5) {
        const float r0 = lane_value(v, 0), r1 = lane_value(v, 16), r2 = lane_value(v, 32), r3 = lane_value(v, 48);
        if (log2w == 5) v = (threadIdx.x & 32) ? op(r2, r3) : op(r0, r1);
        else v = op(op(r0, r1), op(r2, r3));
    }
    return v;
}

// Sum over the wave in f64 (two 32-bit DPP moves per step); every lane receives
// the same result.
template <int CTRL>
__device__ __forceinline__ double dpp_mov_f64(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_mov_dpp(int(b), CTRL, 0xf, 0xf, true);
    const int hi = __builtin_amdgcn_mov_dpp(int(b >> 32), CTRL, 0xf, 0xf, true);
    return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}
__device__ __forceinline__ double lane_value_f64(double v, int lane) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane(int(b), lane), hi = __builtin_amdgcn_readlane(int(b >> 32), lane);
    return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_mov_f64<kDppXor1>(v);
    v += dpp_mov_f64<kDppXor2>(v);
    v += dpp_mov_f64<kDppHalfMirror>(v);
    v += dpp_mov_f64<kDppMirror>(v);
    return (lane_value_f64(v, 0) + lane_value_f64(v, 16)) + (lane_value_f64(v, 32) + lane_value_f64(v, 48));
}

// Sum over aligned groups of W lanes (W = 1, 2, 4, 8, 16) in f64; every lane of a group
// receives the same, bitwise identical result.
template <int W>
__device__ __forceinline__ double group_sum_f64(double v) {
    if constexpr (W >= 2) v += dpp_mov_f64<kDppXor1>(v);
    if constexpr (W >= 4) v += dpp_mov_f64<kDppXor2>(v);
    if constexpr (W >= 8) v += dpp_mov_f64<kDppHalfMirror>(v);
    if constexpr (W >= 16) v += dpp_mov_f64<kDppMirror>(v);
    static_assert(W <= 16, "groups of at most 16 lanes");
    return v;
}

struct OpAdd {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

template <int W>
__device__ __forceinline__ float group_sum(float v) {
    constexpr int l2 = W >= 64 ? 6 : W >= 32 ? 5 : W >= 16 ? 4 : W >= 8 ? 3 : W >= 4 ? 2 : W >= 2 ? 1 : 0;
    return group_reduce(v, l2, OpAdd{});
}

__device__ __forceinline__ float group_sum_dyn(float v, int log2w) { return group_reduce(v, log2w, OpAdd{}); }

__device__ __forceinline__ float wave_sum(float v) { return group_reduce(v, 6, OpAdd{}); }

__device__ __forceinline__ float wave_max(float v) { return group_reduce(v, 6, OpMax{}); }

// (value, index) argmax step: larger value wins, ties go to the lower index.
__device__ __forceinline__ void argmax_merge(float &v, uint32_t &i, float ov, uint32_t oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__device__ __forceinline__ void wave_argmax(float &v, uint32_t &i) {
    auto step = [&](float ov, uint32_t oi) { argmax_merge(v, i, ov, oi); };
    step(dpp_mov<kDppXor1>(v), dpp_mov<kDppXor1>(i));
    step(dpp_mov<kDppXor2>(v), dpp_mov<kDppXor2>(i));
    step(dpp_mov<kDppHalfMirror>(v), dpp_mov<kDppHalfMirror>(i));
    step(dpp_mov<kDppMirror>(v), dpp_mov<kDppMirror>(i));
    float rv[4];
    uint32_t ri[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        rv[r] = lane_value(v, 16 * r);
        ri[r] = uint32_t(__builtin_amdgcn_readlane(int(i), 16 * r));
    }
    v = rv[0];
    i = ri[0];
#pragma unroll
    for (int r = 1; r < 4; ++r) argmax_merge(v, i, rv[r], ri[r]);
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

__device__ __forceinline__ void add4(float4 &a, const float4 &b) {
    a.x += b.x;
    a.y += b.y;
    a.z += b.z;
    a.w += b.w;
}

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld4(const float *p, int f) { return reinterpret_cast<const float4 *>(p)[f]; }

// Fragment order: the X inputs of the decode GEMMs laid out as their A operand reads
// them.  The 4 values x[m][4g .. 4g + 3] form one 16-byte fragment (4 f32 of the
// residual stream, or split [hi0..hi3 | lo0..lo3] with hi = f16(x), lo = f16(x - hi));
// rows go in tiles of 16 (padded), K in slices of 16 columns, and within a slice the
// fragment of (row r, column group q) is number 16 q + r.  A load instruction of a
// decode GEMM (64 lanes, lane 16 q + r) then reads 1 KB of contiguous memory (slices of
// 16) or four 256-byte runs (slices of 32), whole cache lines, where row-major X gives
// it 64 bytes of each of 16 rows (half of every line it touches: measured about half the
// rate, 256 KB per workgroup in 15.2 us against 8.3 us).  Index of the fragment holding
// column k (k % 4 == 0) of row m, for rows of K columns.
__host__ __device__ __forceinline__ size_t frag_index(int m, int k, int K) {
    return (size_t(m >> 4) * size_t(K >> 4) + size_t(k >> 4)) * 64 + size_t((k >> 2) & 3) * 16 + size_t(m & 15);
}

// Eight consecutive values of a K or V cache row: f16 (one 16-byte load) or f32 (two).
// unpack yields them as f32, zeros where keep is false (a masked key's value must not
// reach the sum even as 0 * NaN).
template <typename KT>
struct Kv8;
template <>
struct Kv8<__half> {
    uint4 w;
    __device__ __forceinline__ void load(const __half *p) { w = *reinterpret_cast<const uint4 *>(p); }
    __device__ __forceinline__ void unpack(float (&o)[8], bool keep = true) const {
        const uint32_t a[4] = {keep ? w.x : 0u, keep ? w.y : 0u, keep ? w.z : 0u, keep ? w.w : 0u};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            o[2 * j] = h2f(a[j]);
            o[2 * j + 1] = h2f(a[j] >> 16);
        }
    }
};
template <>
struct Kv8<float> {
    float4 a, b;
    __device__ __forceinline__ void load(const float *p) {
        a = ld4(p, 0);
        b = ld4(p, 1);
    }
    __device__ __forceinline__ void unpack(float (&o)[8], bool keep = true) const {
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = keep ? v[j] : 0.f;
    }
};

// f(std::integral_constant<int, I>) for I = 0 .. N - 1: loop indices that are constants
// from the start (register arrays indexed by them stay in registers)
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// ---- LayerNorm statistics in f64 (biased variance, eps inside the root) ----------
// The f64 sums of a float4's values and squares, paired as the fused step's prologue.
__device__ __forceinline__ void ln_acc(const float4 &v, double &s1, double &s2) {
    const double x0 = v.x, x1 = v.y, x2 = v.z, x3 = v.w;
    s1 += (x0 + x1) + (x2 + x3);
    s2 += (x0 * x0 + x1 * x1) + (x2 * x2 + x3 * x3);
}

// Mean and 1 / sqrt(var + eps) of a row of d values from the wave's lanes' f64 sums of
// x and x^2 (one pass); every lane receives them.
__device__ __forceinline__ void wave_ln_stats(double s1, double s2, int d, float eps, float &mean, float &rstd) {
    s1 = wave_sum_f64(s1);
    s2 = wave_sum_f64(s2);
    const double mu = s1 / d;
    const double var = fmax(s2 / d - mu * mu, 0.0);
    mean = float(mu);
    rstd = float(1.0 / sqrt(var + double(eps)));
}

__device__ __forceinline__ float4 ln_apply(const float4 &v, float mean, float rstd, const float4 &g, const float4 &b) {
    return make_float4((v.x - mean) * rstd * g.x + b.x, (v.y - mean) * rstd * g.y + b.y,
                       (v.z - mean) * rstd * g.z + b.z, (v.w - mean) * rstd * g.w + b.w);
}

// Row LayerNorm by one wave, no LDS and no barrier: lane l holds the float4 slots
// f = l + 64 j (j < NJ, so d <= 256 NJ, d % 4 == 0) of the row in registers between the
// statistics and the normalization.  form(f) returns slot f of the input row; keep(f, v)
// sees it first (a residual kernel stores it there).  out may point to global memory
// or LDS.
template <int NJ, class Form, class Keep>
__device__ __forceinline__ void wave_row_layernorm(int d, Form form, Keep keep, const float *g, const float *b,
                                                   float eps, float *out) {
    const int lane = threadIdx.x & 63, nf = d >> 2;
    // gamma and beta requested first (slots past the row re-read its last one), so that
    // they arrive with the row instead of one round trip after its statistics
    float4 gv[NJ], bv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int f = min(lane + 64 * j, nf - 1);
        gv[j] = ld4(g, f);
        bv[j] = ld4(b, f);
    }
    float4 v[NJ];
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int f = lane + 64 * j;
        if (f < nf) {
            v[j] = form(f);
            keep(f, v[j]);
            ln_acc(v[j], s1, s2);
        }
    }
    float mean, rstd;
    wave_ln_stats(s1, s2, d, eps, mean, rstd);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int f = lane + 64 * j;
        if (f < nf) reinterpret_cast<float4 *>(out)[f] = ln_apply(v[j], mean, rstd, gv[j], bv[j]);
    }
}

struct NoKeep {
    __device__ void operator()(int, const float4 &) const {}
};

// Row LayerNorm by a workgroup of 256 threads: thread t holds the float4 slots
// f = t + 256 c (c < NC, d <= 1024 NC) in registers; the f64 sums go across the wave
// with DPP and across the four waves through red[8] (LDS, fixed order), as the fused
// step's prologue does.  Every thread of the workgroup must call it (two barriers).
template <int NC, class Form, class Keep>
__device__ __forceinline__ void workgroup_row_layernorm(int d, Form form, Keep keep, const float *g, const float *b,
                                                        float eps, float *out, double *red) {
    const int t = threadIdx.x, nf = d >> 2, lane = t & 63, w = t >> 6;
    // gamma and beta are read after the statistics: requested first, they measured slower
    // in the LM-head GEMV's prologue (37.0 -> 37.6 us; 4 more registers, and the weights
    // requested before the prologue are ahead of them either way)
    float4 v[NC];
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int f = t + 256 * c;
        if (f < nf) {
            v[c] = form(f);
            keep(f, v[c]);
            ln_acc(v[c], s1, s2);
        }
    }
    s1 = wave_sum_f64(s1);
    s2 = wave_sum_f64(s2);
    if (lane == 0) {
        red[w] = s1;
        red[4 + w] = s2;
    }
    __syncthreads();
    const double mu = ((red[0] + red[1]) + (red[2] + red[3])) / d;
    const double var = fmax(((red[4] + red[5]) + (red[6] + red[7])) / d - mu * mu, 0.0);
    __syncthreads();  // red is free for the next row
    const float mean = float(mu), rstd = float(1.0 / sqrt(var + double(eps)));
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int f = t + 256 * c;
        if (f < nf) reinterpret_cast<float4 *>(out)[f] = ln_apply(v[c], mean, rstd, ld4(g, f), ld4(b, f));
    }
}

// Largest row a wave normalizes (16 float4 slots per lane).
constexpr int kWaveLnMaxD = 4096;

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

// 6-bit (scale, min) pair j of a Q4_K / Q5_K block as integers; s0..s2 are the 12 scale bytes.
__device__ __forceinline__ void k4_scale_min_u(int j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &a,
                                               uint32_t &b) {
    const uint32_t w[3] = {s0, s1, s2};
    auto byte = [&](int k) { return (w[k >> 2] >> (8 * (k & 3))) & 0xffu; };
    if (j < 4) {
        a = byte(j) & 63;
        b = byte(j + 4) & 63;
    } else {
        a = (byte(j + 4) & 0xf) | ((byte(j - 4) >> 6) << 4);
        b = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
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
