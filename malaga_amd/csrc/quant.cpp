// Block quantizers and dequantizers for the GGUF formats malaga writes.
//
// The reference quantizes with candle-core 0.11 `QTensor::quantize`
// (src/convert.rs:128-136), which is not vendored.  The quantizers here follow
// ggml's published reference algorithms (quantize_row_q8_0 / q4_K / q5_K /
// q6_K with make_qkx2_quants and make_qx_quants).  Parity of the decode path
// is anchored on the GGUF bytes, not on the quantizer: the oracle and the GPU
// both dequantize the same blocks.
#include "quant.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

namespace mlg {

bool type_info(uint32_t type, TypeInfo *o) {
    switch (type) {
    case GGML_F32: *o = {1, 4}; return true;
    case GGML_F16: *o = {1, 2}; return true;
    case GGML_BF16: *o = {1, 2}; return true;
    case GGML_Q8_0: *o = {32, 34}; return true;
    case GGML_Q4_K: *o = {256, 144}; return true;
    case GGML_Q5_K: *o = {256, 176}; return true;
    case GGML_Q6_K: *o = {256, 210}; return true;
    default: return false;
    }
}

const char *type_name(uint32_t type) {
    switch (type) {
    case GGML_F32: return "f32";
    case GGML_F16: return "f16";
    case GGML_BF16: return "bf16";
    case GGML_Q8_0: return "q8_0";
    case GGML_Q4_K: return "q4_K";
    case GGML_Q5_K: return "q5_K";
    case GGML_Q6_K: return "q6_K";
    default: return "?";
    }
}

int64_t type_bytes(uint32_t type, int64_t n) {
    TypeInfo t;
    if (!type_info(type, &t) || n % t.block_elems) return -1;
    return n / t.block_elems * t.block_bytes;
}

uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return uint16_t(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return uint16_t(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return uint16_t(sign);
        const uint32_t e = ax >> 23, mant = (ax & 0x7fffffu) | 0x800000u, shift = 126 - e;
        uint32_t q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return uint16_t(sign | q);
    }
    uint32_t r = ax - 0x38000000u;
    const uint32_t lo = r & 0x1fffu;
    r >>= 13;
    if (lo > 0x1000u || (lo == 0x1000u && (r & 1))) r++;
    return uint16_t(sign | r);
}

float f16_to_f32(uint16_t h) {
    const uint32_t s = uint32_t(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else {
            float f = float(m) * (1.0f / 16777216.0f);
            std::memcpy(&bits, &f, 4);
            bits |= s;
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t f32_to_bf16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return uint16_t((x >> 16) | 0x40);
    x += 0x7fffu + ((x >> 16) & 1);
    return uint16_t(x >> 16);
}

float bf16_to_f32(uint16_t h) {
    uint32_t b = uint32_t(h) << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

namespace {

constexpr float kGroupMaxEps = 1e-15f;

// Round half to even via the 1.5*2^23 trick (ggml's nearest_int).
inline int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    std::memcpy(&i, &val, 4);
    return (i & 0x007fffff) - 0x00400000;
}

// Weighted asymmetric quantization of n values to [0, nmax]; returns the scale,
// *the_min receives -min (ggml make_qkx2_quants).
float make_qkx2_quants(int n, int nmax, const float *x, const float *w, uint8_t *L, float *the_min, uint8_t *Laux,
                       float rmin, float rdelta, int nstep, bool use_mad) {
    float min = x[0], max = x[0];
    float sum_w = w[0], sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_mad = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        L[i] = uint8_t(std::max(0, std::min(nmax, l)));
        float diff = scale * L[i] + min - x[i];
        diff = use_mad ? std::fabs(diff) : diff * diff;
        best_mad += w[i] * diff;
    }
    if (nstep < 1) {
        *the_min = -min;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = std::max(0, std::min(nmax, l));
            Laux[i] = uint8_t(l);
            sum_l += w[i] * l;
            sum_l2 += w[i] * l * l;
            sum_xl += w[i] * l * x[i];
        }
        float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = use_mad ? std::fabs(diff) : diff * diff;
                mad += w[i] * diff;
            }
            if (mad < best_mad) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_mad = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

// Symmetric quantization to [-nmax, nmax-1] with an RMSE search (ggml make_qx_quants,
// rmse_type 1, no importance weights).  L receives values offset by nmax.
float make_qx_quants(int n, int nmax, const float *x, int8_t *L) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = std::fabs(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < kGroupMaxEps) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = std::max(-nmax, std::min(nmax - 1, l));
        L[i] = int8_t(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = std::max(-nmax, std::min(nmax - 1, l));
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                L[i] = int8_t(nmax + std::max(-nmax, std::min(nmax - 1, l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

inline void put16(uint8_t *p, uint16_t v) {
    p[0] = uint8_t(v);
    p[1] = uint8_t(v >> 8);
}
inline uint16_t get16(const uint8_t *p) { return uint16_t(p[0] | (p[1] << 8)); }

inline void scale_min_k4(int j, const uint8_t *q, int *d, int *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// d = amax / 127, q = round(x / d) (round half away from zero).
void quant_q8_0(const float *x, uint8_t *y) {
    float amax = 0;
    for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
    const float d = amax / 127.f, id = d != 0.f ? 1.f / d : 0.f;
    put16(y, f32_to_f16(d));
    for (int i = 0; i < 32; ++i) y[2 + i] = uint8_t(int8_t(std::round(x[i] * id)));
}

// Packs 8 (scale, min) 6-bit pairs into the 12-byte K-quant table.
void pack_scales_k4(const uint8_t *ls, const uint8_t *lm, uint8_t *s) {
    std::memset(s, 0, 12);
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            s[j] = ls[j];
            s[j + 4] = lm[j];
        } else {
            s[j + 4] = uint8_t((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
            s[j - 4] |= uint8_t((ls[j] >> 4) << 6);
            s[j - 0] |= uint8_t((lm[j] >> 4) << 6);
        }
    }
}

// Shared by Q4_K (nmax 15) and Q5_K (nmax 31): per-32 scale/min search, then the
// 6-bit scale table and the final integer levels.  L receives levels 0..nmax.
void k4_levels(const float *x, int nmax, uint8_t *scales12, uint16_t *d16, uint16_t *dmin16, uint8_t *L) {
    float weights[32], mins[8], scales[8];
    uint8_t Laux[32];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = std::sqrt(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + std::fabs(x[32 * j + l]);
        scales[j] = make_qkx2_quants(32, nmax, x + 32 * j, weights, L + 32 * j, &mins[j], Laux,
                                     nmax == 15 ? -1.f : -0.5f, 0.1f, nmax == 15 ? 20 : 15, false);
        max_scale = std::max(max_scale, scales[j]);
        max_min = std::max(max_min, mins[j]);
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    uint8_t ls[8], lm[8];
    for (int j = 0; j < 8; ++j) {
        ls[j] = uint8_t(std::min(63, nearest_int(inv_scale * scales[j])));
        lm[j] = uint8_t(std::min(63, nearest_int(inv_min * mins[j])));
    }
    pack_scales_k4(ls, lm, scales12);
    *d16 = f32_to_f16(max_scale / 63.f);
    *dmin16 = f32_to_f16(max_min / 63.f);
    for (int j = 0; j < 8; ++j) {
        int sc, m;
        scale_min_k4(j, scales12, &sc, &m);
        const float d = f16_to_f32(*d16) * sc;
        if (!d) continue;
        const float dm = f16_to_f32(*dmin16) * m;
        for (int ii = 0; ii < 32; ++ii) {
            const int l = nearest_int((x[32 * j + ii] + dm) / d);
            L[32 * j + ii] = uint8_t(std::max(0, std::min(nmax, l)));
        }
    }
}

void quant_q4_k(const float *x, uint8_t *y) {
    uint8_t L[256];
    uint16_t d, dmin;
    std::memset(L, 0, sizeof L);
    k4_levels(x, 15, y + 4, &d, &dmin, L);
    put16(y, d);
    put16(y + 2, dmin);
    uint8_t *q = y + 16;
    for (int j = 0; j < 256; j += 64, q += 32)
        for (int l = 0; l < 32; ++l) q[l] = uint8_t(L[j + l] | (L[j + l + 32] << 4));
}

void quant_q5_k(const float *x, uint8_t *y) {
    uint8_t L[256];
    uint16_t d, dmin;
    std::memset(L, 0, sizeof L);
    k4_levels(x, 31, y + 4, &d, &dmin, L);
    put16(y, d);
    put16(y + 2, dmin);
    uint8_t *qh = y + 16, *ql = y + 48;
    std::memset(qh, 0, 32);
    uint8_t m1 = 1, m2 = 2;
    for (int n = 0; n < 256; n += 64, ql += 32, m1 <<= 2, m2 <<= 2) {
        for (int j = 0; j < 32; ++j) {
            int l1 = L[n + j];
            if (l1 > 15) { l1 -= 16; qh[j] |= m1; }
            int l2 = L[n + j + 32];
            if (l2 > 15) { l2 -= 16; qh[j] |= m2; }
            ql[j] = uint8_t(l1 | (l2 << 4));
        }
    }
}

void quant_q6_k(const float *x, uint8_t *y) {
    int8_t L[256];
    float scales[16];
    float max_scale = 0, max_abs_scale = 0;
    for (int ib = 0; ib < 16; ++ib) {
        const float scale = make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib);
        scales[ib] = scale;
        const float abs_scale = std::fabs(scale);
        if (abs_scale > max_abs_scale) {
            max_abs_scale = abs_scale;
            max_scale = scale;
        }
    }
    std::memset(y, 0, 210);
    if (max_abs_scale < kGroupMaxEps) return;  // all-zero block, d = 0
    const float iscale = -128.f / max_scale;
    put16(y + 208, f32_to_f16(1 / iscale));
    int8_t *sc = reinterpret_cast<int8_t *>(y + 192);
    for (int ib = 0; ib < 16; ++ib) sc[ib] = int8_t(std::min(127, nearest_int(iscale * scales[ib])));
    for (int j = 0; j < 16; ++j) {
        const float d = f16_to_f32(get16(y + 208)) * sc[j];
        if (!d) continue;
        for (int ii = 0; ii < 16; ++ii) {
            int l = nearest_int(x[16 * j + ii] / d);
            l = std::max(-32, std::min(31, l));
            L[16 * j + ii] = int8_t(l + 32);
        }
    }
    uint8_t *ql = y, *qh = y + 128;
    for (int j = 0; j < 256; j += 128, ql += 64, qh += 32) {
        for (int l = 0; l < 32; ++l) {
            const uint8_t q1 = L[j + l + 0] & 0xF, q2 = L[j + l + 32] & 0xF;
            const uint8_t q3 = L[j + l + 64] & 0xF, q4 = L[j + l + 96] & 0xF;
            ql[l + 0] = uint8_t(q1 | (q3 << 4));
            ql[l + 32] = uint8_t(q2 | (q4 << 4));
            qh[l] = uint8_t((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                            ((L[j + l + 96] >> 4) << 6));
        }
    }
}

}  // namespace

bool quantize(uint32_t type, const float *x, int64_t n, void *out) {
    TypeInfo ti;
    if (!type_info(type, &ti) || n % ti.block_elems) return false;
    uint8_t *y = static_cast<uint8_t *>(out);
    const int64_t nb = n / ti.block_elems;
    switch (type) {
    case GGML_F32: std::memcpy(out, x, size_t(n) * 4); return true;
    case GGML_F16:
        for (int64_t i = 0; i < n; ++i) put16(y + 2 * i, f32_to_f16(x[i]));
        return true;
    case GGML_BF16:
        for (int64_t i = 0; i < n; ++i) put16(y + 2 * i, f32_to_bf16(x[i]));
        return true;
    case GGML_Q8_0:
        for (int64_t b = 0; b < nb; ++b) quant_q8_0(x + 32 * b, y + 34 * b);
        return true;
    case GGML_Q4_K:
        for (int64_t b = 0; b < nb; ++b) quant_q4_k(x + 256 * b, y + 144 * b);
        return true;
    case GGML_Q5_K:
        for (int64_t b = 0; b < nb; ++b) quant_q5_k(x + 256 * b, y + 176 * b);
        return true;
    case GGML_Q6_K:
        for (int64_t b = 0; b < nb; ++b) quant_q6_k(x + 256 * b, y + 210 * b);
        return true;
    default: return false;
    }
}

bool dequantize(uint32_t type, const void *in, int64_t n, float *y) {
    TypeInfo ti;
    if (!type_info(type, &ti) || n % ti.block_elems) return false;
    const uint8_t *p = static_cast<const uint8_t *>(in);
    const int64_t nb = n / ti.block_elems;
    switch (type) {
    case GGML_F32: std::memcpy(y, in, size_t(n) * 4); return true;
    case GGML_F16:
        for (int64_t i = 0; i < n; ++i) y[i] = f16_to_f32(get16(p + 2 * i));
        return true;
    case GGML_BF16:
        for (int64_t i = 0; i < n; ++i) y[i] = bf16_to_f32(get16(p + 2 * i));
        return true;
    case GGML_Q8_0:
        for (int64_t b = 0; b < nb; ++b, p += 34) {
            const float d = f16_to_f32(get16(p));
            for (int l = 0; l < 32; ++l) *y++ = d * float(int8_t(p[2 + l]));
        }
        return true;
    case GGML_Q4_K:
        for (int64_t b = 0; b < nb; ++b, p += 144) {
            const float d = f16_to_f32(get16(p)), dmin = f16_to_f32(get16(p + 2));
            const uint8_t *q = p + 16;
            for (int g = 0; g < 4; ++g, q += 32, y += 64) {
                int s0, m0, s1, m1;
                scale_min_k4(2 * g, p + 4, &s0, &m0);
                scale_min_k4(2 * g + 1, p + 4, &s1, &m1);
                const float d0 = d * s0, mm0 = dmin * m0, d1 = d * s1, mm1 = dmin * m1;
                for (int l = 0; l < 32; ++l) y[l] = d0 * (q[l] & 0xF) - mm0;
                for (int l = 0; l < 32; ++l) y[32 + l] = d1 * (q[l] >> 4) - mm1;
            }
        }
        return true;
    case GGML_Q5_K:
        for (int64_t b = 0; b < nb; ++b, p += 176) {
            const float d = f16_to_f32(get16(p)), dmin = f16_to_f32(get16(p + 2));
            const uint8_t *qh = p + 16, *ql = p + 48;
            for (int g = 0; g < 4; ++g, ql += 32, y += 64) {
                int s0, m0, s1, m1;
                scale_min_k4(2 * g, p + 4, &s0, &m0);
                scale_min_k4(2 * g + 1, p + 4, &s1, &m1);
                const float d0 = d * s0, mm0 = dmin * m0, d1 = d * s1, mm1 = dmin * m1;
                for (int l = 0; l < 32; ++l) y[l] = d0 * ((ql[l] & 0xF) + (((qh[l] >> (2 * g)) & 1) << 4)) - mm0;
                for (int l = 0; l < 32; ++l) y[32 + l] = d1 * ((ql[l] >> 4) + (((qh[l] >> (2 * g + 1)) & 1) << 4)) - mm1;
            }
        }
        return true;
    case GGML_Q6_K:
        for (int64_t b = 0; b < nb; ++b, p += 210) {
            const uint8_t *ql = p, *qh = p + 128;
            const int8_t *sc = reinterpret_cast<const int8_t *>(p + 192);
            const float d = f16_to_f32(get16(p + 208));
            for (int h = 0; h < 2; ++h, ql += 64, qh += 32, sc += 8, y += 128)
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    y[l] = d * sc[is] * (int((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32);
                    y[l + 32] = d * sc[is + 2] * (int((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                    y[l + 64] = d * sc[is + 4] * (int((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                    y[l + 96] = d * sc[is + 6] * (int((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
                }
        }
        return true;
    default: return false;
    }
}

bool quantize_rows(uint32_t type, const float *x, int64_t rows, int64_t k, void *out) {
    const int64_t rb = type_bytes(type, k);
    if (rb < 0) return false;
    bool ok = true;
#pragma omp parallel for schedule(dynamic, 64) reduction(&& : ok)
    for (int64_t r = 0; r < rows; ++r) ok = quantize(type, x + r * k, k, static_cast<uint8_t *>(out) + r * rb) && ok;
    return ok;
}

}  // namespace mlg
