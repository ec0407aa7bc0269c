#include "gguf.hpp"

#include <cstdio>
#include <cstring>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace mlg {

namespace {

struct Reader {
    const uint8_t *p, *end;
    bool bad = false;
    uint64_t u(int n) {
        if (bad || p + n > end) { bad = true; return 0; }
        uint64_t v = 0;
        for (int i = 0; i < n; ++i) v |= uint64_t(p[i]) << (8 * i);
        p += n;
        return v;
    }
    std::string str() {
        const uint64_t n = u(8);
        if (bad || uint64_t(end - p) < n) { bad = true; return {}; }
        std::string s(reinterpret_cast<const char *>(p), size_t(n));
        p += n;
        return s;
    }
};

bool read_value(Reader &r, uint32_t type, GgufValue &v, int depth) {
    v.type = type;
    switch (type) {
    case GV_U8: case GV_BOOL: v.u = r.u(1); break;
    case GV_I8: v.u = uint64_t(int64_t(int8_t(r.u(1)))); break;
    case GV_U16: v.u = r.u(2); break;
    case GV_I16: v.u = uint64_t(int64_t(int16_t(r.u(2)))); break;
    case GV_U32: v.u = r.u(4); break;
    case GV_I32: v.u = uint64_t(int64_t(int32_t(r.u(4)))); break;
    case GV_U64: case GV_I64: v.u = r.u(8); break;
    case GV_F32: { uint32_t b = uint32_t(r.u(4)); float f; std::memcpy(&f, &b, 4); v.f = f; break; }
    case GV_F64: { uint64_t b = r.u(8); std::memcpy(&v.f, &b, 8); break; }
    case GV_STRING: v.s = r.str(); break;
    case GV_ARRAY: {
        if (depth > 2) return false;
        v.elem_type = uint32_t(r.u(4));
        const uint64_t n = r.u(8);
        if (r.bad || n > uint64_t(r.end - r.p)) return false;
        v.arr.resize(size_t(n));
        for (auto &e : v.arr)
            if (!read_value(r, v.elem_type, e, depth + 1)) return false;
        break;
    }
    default: return false;
    }
    return !r.bad;
}

void put(std::vector<uint8_t> &o, uint64_t v, int n) {
    for (int i = 0; i < n; ++i) o.push_back(uint8_t(v >> (8 * i)));
}
void put_str(std::vector<uint8_t> &o, const std::string &s) {
    put(o, s.size(), 8);
    o.insert(o.end(), s.begin(), s.end());
}
void put_value(std::vector<uint8_t> &o, const GgufValue &v) {
    switch (v.type) {
    case GV_U8: case GV_I8: case GV_BOOL: put(o, v.u, 1); break;
    case GV_U16: case GV_I16: put(o, v.u, 2); break;
    case GV_U32: case GV_I32: put(o, v.u, 4); break;
    case GV_U64: case GV_I64: put(o, v.u, 8); break;
    case GV_F32: { float f = float(v.f); uint32_t b; std::memcpy(&b, &f, 4); put(o, b, 4); break; }
    case GV_F64: { uint64_t b; std::memcpy(&b, &v.f, 8); put(o, b, 8); break; }
    case GV_STRING: put_str(o, v.s); break;
    case GV_ARRAY:
        put(o, v.elem_type, 4);
        put(o, v.arr.size(), 8);
        for (auto &e : v.arr) put_value(o, e);
        break;
    }
}

}  // namespace

GgufFile::~GgufFile() {
    if (map_) munmap(map_, size_);
}

std::string GgufFile::open(const std::string &path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return "cannot open " + path;
    struct stat st;
    if (fstat(fd, &st) != 0) { ::close(fd); return "cannot stat " + path; }
    size_ = size_t(st.st_size);
    void *m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) return "cannot map " + path;
    map_ = static_cast<uint8_t *>(m);
    Reader r{map_, map_ + size_};
    if (r.u(4) != 0x46554747u) return path + ": not a GGUF file";
    const uint32_t version = uint32_t(r.u(4));
    if (version < 2 || version > 3) return path + ": unsupported GGUF version " + std::to_string(version);
    const uint64_t nt = r.u(8), nkv = r.u(8);
    if (r.bad || nt > (1u << 24) || nkv > (1u << 24)) return path + ": corrupt header";
    for (uint64_t i = 0; i < nkv; ++i) {
        std::string key = r.str();
        const uint32_t t = uint32_t(r.u(4));
        GgufValue v;
        if (r.bad || !read_value(r, t, v, 0)) return path + ": corrupt metadata";
        if (key == "general.alignment" && v.is_int() && v.u) align_ = v.u;
        kv_.emplace_back(std::move(key), std::move(v));
    }
    for (uint64_t i = 0; i < nt; ++i) {
        GgufTensorInfo ti;
        ti.name = r.str();
        const uint32_t nd = uint32_t(r.u(4));
        if (r.bad || nd < 1 || nd > 4) return path + ": corrupt tensor info";
        for (uint32_t d = 0; d < nd; ++d) ti.ne.push_back(r.u(8));
        ti.type = uint32_t(r.u(4));
        ti.offset = r.u(8);
        if (r.bad) return path + ": corrupt tensor info";
        tindex_[ti.name] = tensors_.size();
        tensors_.push_back(std::move(ti));
    }
    size_t pos = size_t(r.p - map_);
    pos = (pos + align_ - 1) / align_ * align_;
    data_ = map_ + pos;
    for (auto &t : tensors_)
        if (pos + t.offset > size_) return path + ": tensor " + t.name + " past end of file";
    return {};
}

const GgufValue *GgufFile::get(const std::string &key) const {
    for (auto &kv : kv_)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

const GgufTensorInfo *GgufFile::tensor(const std::string &name) const {
    auto it = tindex_.find(name);
    return it == tindex_.end() ? nullptr : &tensors_[it->second];
}

std::string gguf_write(const std::string &path, const std::vector<std::pair<std::string, GgufValue>> &kv,
                       const std::vector<GgufOutTensor> &tensors) {
    const uint64_t align = 32;
    std::vector<uint8_t> head;
    put(head, 0x46554747u, 4);
    put(head, 3, 4);
    put(head, tensors.size(), 8);
    put(head, kv.size(), 8);
    for (auto &e : kv) {
        put_str(head, e.first);
        put(head, e.second.type, 4);
        put_value(head, e.second);
    }
    uint64_t off = 0;
    for (auto &t : tensors) {
        put_str(head, t.name);
        put(head, t.ne.size(), 4);
        for (auto d : t.ne) put(head, d, 8);
        put(head, t.type, 4);
        put(head, off, 8);
        off += (t.bytes.size() + align - 1) / align * align;
    }
    while (head.size() % align) head.push_back(0);
    const std::string tmp = path + ".partial";
    FILE *f = std::fopen(tmp.c_str(), "wb");
    if (!f) return "cannot create " + tmp;
    bool ok = std::fwrite(head.data(), 1, head.size(), f) == head.size();
    static const uint8_t zeros[32] = {};
    for (auto &t : tensors) {
        if (!ok) break;
        ok = std::fwrite(t.bytes.data(), 1, t.bytes.size(), f) == t.bytes.size();
        const size_t pad = (align - t.bytes.size() % align) % align;
        if (ok && pad) ok = std::fwrite(zeros, 1, pad, f) == pad;
    }
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) { std::remove(tmp.c_str()); return "write failed: " + tmp; }
    if (std::rename(tmp.c_str(), path.c_str()) != 0) return "rename failed: " + path;
    return {};
}

}  // namespace mlg
