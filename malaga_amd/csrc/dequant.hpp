// Device dequantization of 16 consecutive values of one weight row (k0 % 16 == 0),
// for the device layouts of DevMatrix (GGUF blocks / split planes).
#pragma once
#include "device.hpp"
#include "quant.hpp"

namespace mlg {

template <int T>
__device__ __forceinline__ void dequant16(const uint8_t *q, const uint8_t *s, const uint8_t *dp, int K, int row,
                                          int k0, float *out) {
    if constexpr (T == GGML_Q4_K || T == GGML_Q5_K) {
        constexpr int BB = T == GGML_Q4_K ? 144 : 176;
        const int nb = K >> 8, j = k0 >> 8, kk = k0 & 255, sb = kk >> 5, l0 = kk & 31, g = sb >> 1, hi = sb & 1;
        const uint8_t *blk = q + (size_t(row) * nb + j) * BB;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
        const float d = h2f(hdr.x), dmin = h2f(hdr.x >> 16);
        const uint32_t sw[3] = {hdr.y, hdr.z, hdr.w};
        auto byte = [&](int k) { return (sw[k >> 2] >> (8 * (k & 3))) & 0xffu; };
        uint32_t sc, m;
        if (sb < 4) {
            sc = byte(sb) & 63;
            m = byte(sb + 4) & 63;
        } else {
            sc = (byte(sb + 4) & 0xf) | ((byte(sb - 4) >> 6) << 4);
            m = (byte(sb + 4) >> 4) | ((byte(sb) >> 6) << 4);
        }
        const float d1 = d * float(sc), m1 = dmin * float(m);
        const uint8_t *qs = blk + (T == GGML_Q4_K ? 16 : 48) + 32 * g + l0;
        const uint4 raw = *reinterpret_cast<const uint4 *>(qs);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        uint32_t hw[4] = {0, 0, 0, 0};
        if constexpr (T == GGML_Q5_K) {
            const uint4 h = *reinterpret_cast<const uint4 *>(blk + 16 + l0);
            hw[0] = h.x; hw[1] = h.y; hw[2] = h.z; hw[3] = h.w;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t byt = (w[e >> 2] >> (8 * (e & 3))) & 0xffu;
            uint32_t v = hi ? (byt >> 4) : (byt & 15u);
            if constexpr (T == GGML_Q5_K) v |= (((hw[e >> 2] >> (8 * (e & 3))) >> (2 * g + hi)) & 1u) << 4;
            out[e] = d1 * float(v) - m1;
        }
    } else if constexpr (T == GGML_Q6_K) {
        const int nb = K >> 8, j = k0 >> 8, kk = k0 & 255, h2 = kk >> 7, rem = kk & 127, grp = rem >> 5, l0 = rem & 31;
        const size_t blk = size_t(row) * nb + j;
        const uint8_t *qp = q + blk * 192;
        const uint4 lq = *reinterpret_cast<const uint4 *>(qp + 64 * h2 + 32 * (grp & 1) + l0);
        const uint4 hq = *reinterpret_cast<const uint4 *>(qp + 128 + 32 * h2 + l0);
        const float d = h2f(*reinterpret_cast<const unsigned short *>(dp + blk * 2));
        const float sc = float(int8_t(s[blk * 16 + 8 * h2 + (l0 >> 4) + 2 * grp]));
        const float ds = d * sc;
        const uint32_t L[4] = {lq.x, lq.y, lq.z, lq.w}, H[4] = {hq.x, hq.y, hq.z, hq.w};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t lb = (L[e >> 2] >> (8 * (e & 3))) & 0xffu, hb = (H[e >> 2] >> (8 * (e & 3))) & 0xffu;
            const uint32_t v = ((grp >= 2 ? (lb >> 4) : (lb & 15u)) | (((hb >> (2 * grp)) & 3u) << 4));
            out[e] = ds * float(int(v) - 32);
        }
    } else if constexpr (T == GGML_Q8_0) {
        const uint4 raw = *reinterpret_cast<const uint4 *>(q + size_t(row) * K + k0);
        const float d = h2f(*reinterpret_cast<const unsigned short *>(dp + (size_t(row) * (K >> 5) + (k0 >> 5)) * 2));
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < 16; ++e) out[e] = d * float(int8_t(w[e >> 2] >> (8 * (e & 3))));
    } else if constexpr (T == GGML_F16) {
        const uint4 *p = reinterpret_cast<const uint4 *>(q + (size_t(row) * K + k0) * 2);
        const uint4 a = p[0], b = p[1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 16; ++e) out[e] = h2f(w[e >> 1] >> (16 * (e & 1)));
    } else {
        const float4 *p = reinterpret_cast<const float4 *>(q + (size_t(row) * K + k0) * 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float4 v = p[u];
            out[4 * u] = v.x;
            out[4 * u + 1] = v.y;
            out[4 * u + 2] = v.z;
            out[4 * u + 3] = v.w;
        }
    }
}

// Runtime-type dispatch helper for kernels templated on the weight type.
#define MLG_DISPATCH_TYPE(type, FN, ...)                               \
    switch (type) {                                                    \
    case GGML_Q4_K: return FN<GGML_Q4_K>(__VA_ARGS__);                \
    case GGML_Q5_K: return FN<GGML_Q5_K>(__VA_ARGS__);                \
    case GGML_Q6_K: return FN<GGML_Q6_K>(__VA_ARGS__);                \
    case GGML_Q8_0: return FN<GGML_Q8_0>(__VA_ARGS__);                \
    case GGML_F16: return FN<GGML_F16>(__VA_ARGS__);                  \
    case GGML_F32: return FN<GGML_F32>(__VA_ARGS__);                  \
    default: return hipErrorInvalidValue;                             \
    }

}  // namespace mlg
