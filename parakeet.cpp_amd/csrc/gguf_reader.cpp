// gguf_reader.cpp -- see gguf_reader.h.
#include "gguf_reader.h"

#include <cstdio>
#include <cstring>
#include <fstream>

namespace parakeet_hip {
namespace gguf {

namespace {

enum : uint32_t {
    T_U8 = 0, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64
};

struct Cursor {
    const uint8_t *p, *end;
    bool ok = true;
    template <class T> T get() {
        T v{};
        if ((size_t)(end - p) < sizeof(T)) { ok = false; return v; }
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || (uint64_t)(end - p) < n) { ok = false; return {}; }
        std::string s(reinterpret_cast<const char *>(p), n);
        p += n;
        return s;
    }
};

size_t scalar_size(uint32_t t) {
    switch (t) {
        case T_U8: case T_I8: case T_BOOL: return 1;
        case T_U16: case T_I16: return 2;
        case T_U32: case T_I32: case T_F32: return 4;
        case T_U64: case T_I64: case T_F64: return 8;
        default: return 0;
    }
}

int64_t read_int(Cursor &c, uint32_t t) {
    switch (t) {
        case T_U8: return c.get<uint8_t>();
        case T_I8: return c.get<int8_t>();
        case T_BOOL: return c.get<uint8_t>() != 0;
        case T_U16: return c.get<uint16_t>();
        case T_I16: return c.get<int16_t>();
        case T_U32: return c.get<uint32_t>();
        case T_I32: return c.get<int32_t>();
        case T_U64: return (int64_t)c.get<uint64_t>();
        case T_I64: return c.get<int64_t>();
        default: c.ok = false; return 0;
    }
}

bool read_value(Cursor &c, uint32_t t, Value &v) {
    v.type = t;
    if (t == T_STR) {
        v.s = c.str();
    } else if (t == T_F32) {
        v.f = c.get<float>();
    } else if (t == T_F64) {
        v.f = c.get<double>();
    } else if (t == T_ARR) {
        v.arr_type = c.get<uint32_t>();
        const uint64_t n = c.get<uint64_t>();
        if (!c.ok) return false;
        // an element takes at least its size in the file (a string its 8-byte
        // length), so a count past what remains is a corrupt header
        const uint64_t left = (uint64_t)(c.end - c.p);
        if (v.arr_type == T_STR) {
            if (n > left / 8) return false;
            v.arr_s.reserve(n);
            for (uint64_t i = 0; i < n && c.ok; ++i) v.arr_s.push_back(c.str());
        } else if (v.arr_type == T_F32 || v.arr_type == T_F64) {
            const size_t sz = scalar_size(v.arr_type);
            if (n > left / sz) return false;
            c.p += n * sz;   // float arrays are not used by the decoder
        } else {
            const size_t sz = scalar_size(v.arr_type);
            if (sz == 0 || n > left / sz) return false;
            v.arr_i.reserve(n);
            for (uint64_t i = 0; i < n && c.ok; ++i) v.arr_i.push_back(read_int(c, v.arr_type));
        }
    } else {
        v.i = read_int(c, t);
    }
    return c.ok;
}

}  // namespace

uint64_t tensor_nbytes(uint32_t type, int64_t n) {
    if (n < 0) return 0;
    const uint64_t blocks = (uint64_t)n / 32;
    const bool whole = n % 32 == 0;
    switch (type) {
        case 0: return 4ull * (uint64_t)n;
        case 1: return 2ull * (uint64_t)n;
        case 2: return whole ? blocks * 18ull : 0;   // q4_0 {f16 d; u8 qs[16]}
        case 6: return whole ? blocks * 22ull : 0;   // q5_0 {f16 d; u8 qh[4]; u8 qs[16]}
        case 8: return whole ? blocks * 34ull : 0;   // q8_0 {f16 d; i8 q[32]}
        default: return 0;
    }
}

int File::open(const std::string &path, std::string &err) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) { err = "cannot open " + path; return 1; }
    const std::streamsize size = f.tellg();
    if (size < 0) { err = "cannot size " + path; return 1; }
    f.seekg(0);
    std::vector<uint8_t> bytes((size_t)size);
    if (!f.read(reinterpret_cast<char *>(bytes.data()), size)) { err = "short read " + path; return 1; }
    if (parse(std::move(bytes), err)) {
        err = path + ": " + err;
        return 1;
    }
    return 0;
}

int File::parse(std::vector<uint8_t> bytes, std::string &err) {
    bytes_ = std::move(bytes);
    kv_.clear();
    tensors_.clear();
    Cursor c{bytes_.data(), bytes_.data() + bytes_.size()};
    if (bytes_.size() < 24 || memcmp(bytes_.data(), "GGUF", 4) != 0) { err = "not GGUF"; return 1; }
    c.p += 4;
    const uint32_t version = c.get<uint32_t>();
    if (version != 2 && version != 3) { err = "unsupported GGUF version"; return 1; }
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv && c.ok; ++i) {
        std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        Value v;
        if (!read_value(c, t, v)) { err = "bad metadata value for " + key; return 1; }
        kv_[key] = std::move(v);
    }
    uint64_t align = 32;
    if (const Value *a = find("general.alignment")) {
        if (a->i < 1 || a->i > (1 << 20)) { err = "bad general.alignment"; return 1; }
        align = (uint64_t)a->i;
    }
    std::vector<Tensor> infos;
    for (uint64_t i = 0; i < n_tensors && c.ok; ++i) {
        Tensor t;
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (nd > 4) { err = "tensor rank > 4"; return 1; }
        for (uint32_t d = 0; d < nd; ++d) {
            const uint64_t v = c.get<uint64_t>();
            if (v > (1ull << 32)) { err = "tensor dimension out of range"; return 1; }
            t.ne.push_back((int64_t)v);
        }
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        infos.push_back(std::move(t));
    }
    if (!c.ok) { err = "truncated GGUF header"; return 1; }
    const uint64_t base = ((uint64_t)(c.p - bytes_.data()) + align - 1) / align * align;
    for (auto &t : infos) {
        int64_t n = 1;
        for (int64_t v : t.ne) {
            n *= v;
            if (n > (1ll << 40)) { err = "tensor " + t.name + " too large"; return 1; }
        }
        t.nbytes = tensor_nbytes(t.type, n);
        const uint64_t size = bytes_.size();
        if (t.offset > size || base > size - t.offset) { err = "tensor " + t.name + " out of file bounds"; return 1; }
        t.offset += base;
        if (t.nbytes == 0 || t.nbytes > size - t.offset) {
            err = "tensor " + t.name + " out of file bounds or of unsupported type";
            return 1;
        }
        t.data = bytes_.data() + t.offset;
        tensors_[t.name] = t;
    }
    return 0;
}

const Value *File::find(const std::string &key) const {
    auto it = kv_.find(key);
    return it == kv_.end() ? nullptr : &it->second;
}

const Tensor *File::tensor(const std::string &name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

uint32_t File::get_u32(const std::string &key, uint32_t def) const {
    const Value *v = find(key);
    return v ? (uint32_t)v->i : def;
}

int32_t File::get_i32(const std::string &key, int32_t def) const {
    const Value *v = find(key);
    return v ? (int32_t)v->i : def;
}

bool File::get_bool(const std::string &key, bool def) const {
    const Value *v = find(key);
    return v ? v->i != 0 : def;
}

std::string File::get_str(const std::string &key, const std::string &def) const {
    const Value *v = find(key);
    return v ? v->s : def;
}

}  // namespace gguf
}  // namespace parakeet_hip
