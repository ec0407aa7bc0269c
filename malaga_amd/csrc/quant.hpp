// ggml block formats used by malaga's GGUF presets (src/convert.rs:25-91, 148-162):
// F32, F16, Q8_0, Q4_K, Q5_K, Q6_K.  Byte layouts are the public GGUF/ggml ones.
#pragma once
#include <cstddef>
#include <cstdint>

namespace mlg {

enum GgmlType : uint32_t {
    GGML_F32 = 0,
    GGML_F16 = 1,
    GGML_Q8_0 = 8,
    GGML_Q4_K = 12,
    GGML_Q5_K = 13,
    GGML_Q6_K = 14,
    GGML_BF16 = 30,
};

struct TypeInfo {
    int block_elems;  // values per block
    int block_bytes;  // bytes per block
};

// false for types this build does not handle
bool type_info(uint32_t type, TypeInfo *out);
const char *type_name(uint32_t type);
// bytes of n values (n must be a multiple of the block size)
int64_t type_bytes(uint32_t type, int64_t n);

uint16_t f32_to_f16(float f);  // IEEE round-to-nearest-even
float f16_to_f32(uint16_t h);
uint16_t f32_to_bf16(float f);  // round-to-nearest-even
float bf16_to_f32(uint16_t h);

// Quantizes / dequantizes n values (a whole number of blocks), single thread.
bool quantize(uint32_t type, const float *x, int64_t n, void *out);
bool dequantize(uint32_t type, const void *in, int64_t n, float *y);

// Row-parallel (OpenMP) quantization of a [rows, k] matrix.
bool quantize_rows(uint32_t type, const float *x, int64_t rows, int64_t k, void *out);

}  // namespace mlg
