// GGUF v3 container: reader (mmap) and writer.
// Public GGUF layout; malaga's metadata keys and tensor names are those of
// src/config.rs:71-116 and src/convert.rs:293-318.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace mlg {

enum GgufValueType : uint32_t {
    GV_U8 = 0, GV_I8 = 1, GV_U16 = 2, GV_I16 = 3, GV_U32 = 4, GV_I32 = 5, GV_F32 = 6, GV_BOOL = 7,
    GV_STRING = 8, GV_ARRAY = 9, GV_U64 = 10, GV_I64 = 11, GV_F64 = 12,
};

struct GgufValue {
    uint32_t type = GV_U32;
    uint64_t u = 0;        // unsigned / bool / signed (two's complement) scalars
    double f = 0;          // float scalars
    std::string s;         // strings
    uint32_t elem_type = 0;           // arrays
    std::vector<GgufValue> arr;

    static GgufValue U32(uint32_t v) { GgufValue x; x.type = GV_U32; x.u = v; return x; }
    static GgufValue Bool(bool v) { GgufValue x; x.type = GV_BOOL; x.u = v; return x; }
    static GgufValue Str(std::string v) { GgufValue x; x.type = GV_STRING; x.s = std::move(v); return x; }
    static GgufValue ArrU32(const std::vector<uint32_t> &v) {
        GgufValue x; x.type = GV_ARRAY; x.elem_type = GV_U32;
        for (uint32_t e : v) x.arr.push_back(U32(e));
        return x;
    }
    bool is_int() const { return type <= GV_I32 || type == GV_BOOL || type == GV_U64 || type == GV_I64; }
};

struct GgufTensorInfo {
    std::string name;
    std::vector<uint64_t> ne;  // ne[0] = innermost (row length)
    uint32_t type = 0;
    uint64_t offset = 0;       // relative to the data section
    int64_t numel() const { int64_t n = 1; for (auto d : ne) n *= int64_t(d); return n; }
};

class GgufFile {
  public:
    GgufFile() = default;
    ~GgufFile();
    GgufFile(const GgufFile &) = delete;
    GgufFile &operator=(const GgufFile &) = delete;

    // Returns an empty string on success, else an error message.
    std::string open(const std::string &path);

    const GgufValue *get(const std::string &key) const;
    const GgufTensorInfo *tensor(const std::string &name) const;
    const uint8_t *tensor_data(const GgufTensorInfo &t) const { return data_ + t.offset; }
    const std::vector<GgufTensorInfo> &tensors() const { return tensors_; }
    const std::vector<std::pair<std::string, GgufValue>> &metadata() const { return kv_; }
    uint64_t alignment() const { return align_; }

  private:
    uint8_t *map_ = nullptr;
    size_t size_ = 0;
    const uint8_t *data_ = nullptr;
    uint64_t align_ = 32;
    std::vector<std::pair<std::string, GgufValue>> kv_;
    std::vector<GgufTensorInfo> tensors_;
    std::map<std::string, size_t> tindex_;
};

struct GgufOutTensor {
    std::string name;
    std::vector<uint64_t> ne;  // ne[0] = row length
    uint32_t type;
    std::vector<uint8_t> bytes;
};

// Writes metadata + tensors (alignment 32) to `path` through `path.partial`
// and a rename, as src/convert.rs:313-317 does.  Returns "" on success.
std::string gguf_write(const std::string &path, const std::vector<std::pair<std::string, GgufValue>> &kv,
                       const std::vector<GgufOutTensor> &tensors);

}  // namespace mlg
