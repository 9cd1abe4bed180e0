// GGUF file reader for the on-disk path of the quantized-matmul library:
// the file is memory-mapped and parsed as src/gguf.rs:201-279 does (magic,
// version, tensor and metadata counts, metadata key/values with nested
// arrays, tensor infos, data section at the next `general.alignment`
// boundary, default 32); tensor byte ranges follow src/gguf.rs:310-334 and
// the block table of src/gguf.rs:366-400. Host code only: tensors are
// uploaded to a device arena by the library's C ABI (rfxq.cpp).
#pragma once
#include <cstdint>
#include <cstring>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

namespace gguf {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read little-endian
constexpr uint64_t kDefaultAlignment = 32;

struct Value {
    enum Kind { UINT, INT, FLOAT, BOOL, STR, ARRAY } kind = UINT;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
    std::vector<Value> arr;
    // the value as an unsigned integer (as_u64 of src/gguf.rs:52-64:
    // unsigned types, non-negative signed ones)
    bool as_u64(uint64_t* out) const {
        if (kind == UINT) return *out = u, true;
        if (kind == INT && i >= 0) return *out = (uint64_t)i, true;
        return false;
    }
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;  // relative to the data section
};

// (elements, bytes) of one block of ggml type `t` (src/gguf.rs:366-400)
inline bool block_dims(uint32_t t, uint64_t* qk, uint64_t* bb) {
    static const struct {
        uint32_t t;
        uint64_t qk, bb;
    } table[] = {
        {0, 1, 4},    {1, 1, 2},      {30, 1, 2},     {28, 1, 8},     {24, 1, 1},     {25, 1, 2},
        {26, 1, 4},   {27, 1, 8},     {8, 32, 34},    {9, 32, 36},    {2, 32, 18},    {3, 32, 20},
        {6, 32, 22},  {7, 32, 24},    {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
        {14, 256, 210}, {15, 256, 292}, {16, 256, 66}, {17, 256, 74},  {22, 256, 82},  {18, 256, 98},
        {21, 256, 110}, {19, 256, 50}, {29, 256, 56},  {23, 256, 136},
    };
    for (const auto& e : table)
        if (e.t == t) {
            *qk = e.qk;
            *bb = e.bb;
            return true;
        }
    return false;
}

class Reader {
  public:
    Reader(const uint8_t* d, size_t n) : d_(d), n_(n) {}
    size_t pos() const { return pos_; }
    bool take(size_t k, const uint8_t** p, std::string* err) {
        if (k > n_ - pos_) {
            *err = "unexpected end of file at offset " + std::to_string(pos_) + " (need " + std::to_string(k) +
                   " more bytes)";
            return false;
        }
        *p = d_ + pos_;
        pos_ += k;
        return true;
    }
    template <class T>
    bool get(T* v, std::string* err) {
        const uint8_t* p;
        if (!take(sizeof(T), &p, err)) return false;
        std::memcpy(v, p, sizeof(T));  // little-endian host
        return true;
    }
    bool str(std::string* s, std::string* err) {
        uint64_t len;
        const uint8_t* p;
        if (!get(&len, err) || !take((size_t)len, &p, err)) return false;
        s->assign(reinterpret_cast<const char*>(p), (size_t)len);
        return true;
    }
    bool scalar(uint32_t t, Value* v, std::string* err) {
        switch (t) {
            case 0: { uint8_t x; if (!get(&x, err)) return false; v->kind = Value::UINT; v->u = x; return true; }
            case 1: { int8_t x; if (!get(&x, err)) return false; v->kind = Value::INT; v->i = x; return true; }
            case 2: { uint16_t x; if (!get(&x, err)) return false; v->kind = Value::UINT; v->u = x; return true; }
            case 3: { int16_t x; if (!get(&x, err)) return false; v->kind = Value::INT; v->i = x; return true; }
            case 4: { uint32_t x; if (!get(&x, err)) return false; v->kind = Value::UINT; v->u = x; return true; }
            case 5: { int32_t x; if (!get(&x, err)) return false; v->kind = Value::INT; v->i = x; return true; }
            case 6: { float x; if (!get(&x, err)) return false; v->kind = Value::FLOAT; v->f = x; return true; }
            case 7: { uint8_t x; if (!get(&x, err)) return false; v->kind = Value::BOOL; v->u = x != 0; return true; }
            case 8: v->kind = Value::STR; return str(&v->s, err);
            case 10: { uint64_t x; if (!get(&x, err)) return false; v->kind = Value::UINT; v->u = x; return true; }
            case 11: { int64_t x; if (!get(&x, err)) return false; v->kind = Value::INT; v->i = x; return true; }
            case 12: { double x; if (!get(&x, err)) return false; v->kind = Value::FLOAT; v->f = x; return true; }
            default: *err = "unsupported GGUF metadata value type " + std::to_string(t); return false;
        }
    }
    // an array body (element type, length, elements; nested arrays carry
    // their own element type and length, src/gguf.rs:505-546)
    bool array(Value* v, std::string* err, int depth = 0) {
        uint32_t et;
        uint64_t len;
        if (depth > 64) return *err = "GGUF arrays nested too deeply", false;
        if (!get(&et, err) || !get(&len, err)) return false;
        v->kind = Value::ARRAY;
        for (uint64_t j = 0; j < len; j++) {
            Value e;
            if (!(et == 9 ? array(&e, err, depth + 1) : scalar(et, &e, err))) return false;
            v->arr.push_back(std::move(e));
        }
        return true;
    }
    bool value(Value* v, std::string* err) {
        uint32_t t;
        if (!get(&t, err)) return false;
        return t == 9 ? array(v, err) : scalar(t, v, err);
    }

  private:
    const uint8_t* d_;
    size_t n_, pos_ = 0;
};

struct File {
    const uint8_t* data = nullptr;
    size_t len = 0;
    uint32_t version = 0;
    uint64_t alignment = kDefaultAlignment;
    uint64_t data_start = 0;
    std::map<std::string, Value> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;

    bool parse(std::string* err) {
        Reader r(data, len);
        uint32_t magic;
        uint64_t nt, nkv;
        if (!r.get(&magic, err)) return false;
        if (magic != kMagic) {
            char b[96];
            std::snprintf(b, sizeof b, "not a GGUF file: magic=%#010x, expected %#010x", magic, kMagic);
            *err = b;
            return false;
        }
        if (!r.get(&version, err) || !r.get(&nt, err) || !r.get(&nkv, err)) return false;
        for (uint64_t i = 0; i < nkv; i++) {
            std::string key;
            Value v;
            if (!r.str(&key, err) || !r.value(&v, err)) return false;
            meta[key] = std::move(v);  // a repeated key keeps the last value
        }
        auto al = meta.find("general.alignment");
        uint64_t a;
        if (al != meta.end() && al->second.as_u64(&a)) alignment = a;
        if (alignment == 0) alignment = 1;
        for (uint64_t i = 0; i < nt; i++) {
            Tensor t;
            uint32_t nd;
            if (!r.str(&t.name, err) || !r.get(&nd, err)) return false;
            for (uint32_t j = 0; j < nd; j++) {
                uint64_t d;
                if (!r.get(&d, err)) return false;
                t.dims.push_back(d);
            }
            if (!r.get(&t.type, err) || !r.get(&t.offset, err)) return false;
            by_name.emplace(t.name, tensors.size());  // the first of a repeated name wins (tensor_info's find)
            tensors.push_back(std::move(t));
        }
        data_start = (r.pos() + alignment - 1) / alignment * alignment;
        if (data_start > len) {
            *err = "data section start " + std::to_string(data_start) + " beyond file length " + std::to_string(len);
            return false;
        }
        return true;
    }

    static uint64_t elements(const Tensor& t) {
        uint64_t n = 1;
        for (uint64_t d : t.dims) n *= d;
        return n;
    }

    // [start, start + bytes) of a tensor's data in the file
    bool range(const Tensor& t, uint64_t* start, uint64_t* bytes, std::string* err) const {
        uint64_t qk, bb;
        if (!block_dims(t.type, &qk, &bb)) {
            *err = "unknown ggml_type=" + std::to_string(t.type) + ": on-disk block size not known to this parser";
            return false;
        }
        *bytes = (elements(t) + qk - 1) / qk * bb;
        *start = data_start + t.offset;
        if (*start < t.offset || *start + *bytes < *start || *start + *bytes > len) {
            *err = "tensor '" + t.name + "' range " + std::to_string(*start) + ".." +
                   std::to_string(*start + *bytes) + " exceeds file length " + std::to_string(len);
            return false;
        }
        return true;
    }
};

}  // namespace gguf
