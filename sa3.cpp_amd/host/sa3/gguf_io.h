// gguf_io.h - a small reader and writer of GGUF version 3 files, enough for adapter checkpoints and
// the trainer-state sidecar: scalar metadata (strings, integers, floats, bools), arrays of u64 and of
// strings (arrays of other element types are skipped when read) and f32 / f16 tensors. The format,
// little-endian throughout:
//   "GGUF", u32 version 3, u64 tensor count, u64 metadata count;
//   metadata: string key, u32 value type, value (string = u64 byte length + bytes);
//   tensor infos: string name, u32 n_dims, u64 ne[n_dims] (ne[0] the contiguous extent), u32 type,
//   u64 offset into the data section;
//   zero padding to `general.alignment` (32 by default), then the data section, every tensor at its
//   offset (each a multiple of the alignment, zero-padded between tensors).
// Metadata and tensors are written in the order they are added, as ggml's gguf writer does.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace sa3 {
namespace gguf {

enum ValueType : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12
};
enum TensorType : uint32_t { kTensorF32 = 0, kTensorF16 = 1 };

constexpr uint32_t kVersion = 3;
constexpr uint64_t kDefaultAlignment = 32;

inline uint64_t align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

// f16 bits -> f32 (exact)
inline float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {   // subnormal: normalise
        int e = 113;
        while (!(man & 0x400u)) {
            man <<= 1;
            --e;
        }
        bits = sign | ((uint32_t)e << 23) | ((man & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

struct Value {
    uint32_t type = kU32;
    std::string s;      // kString
    uint64_t u = 0;     // unsigned integers and bools
    int64_t i = 0;      // signed integers
    double f = 0.0;     // floats
    uint32_t arr_type = 0;               // kArray: element type
    std::vector<uint64_t> au;            // kArray of kU64
    std::vector<std::string> as;         // kArray of kString
};

struct TensorInfo {
    std::string name;
    std::vector<int64_t> ne;
    uint32_t type = kTensorF32;
    uint64_t offset = 0;   // into the data section
    // element count; the parser has checked that every extent is in [1, 2^62) and that their
    // product fits in int64
    int64_t elements() const {
        int64_t n = 1;
        for (int64_t e : ne) n *= e;
        return n;
    }
};

class Writer {
public:
    void set_str(const std::string& k, const std::string& v) {
        Value x;
        x.type = kString;
        x.s = v;
        kv_.push_back({k, x});
    }
    void set_u32(const std::string& k, uint32_t v) {
        Value x;
        x.type = kU32;
        x.u = v;
        kv_.push_back({k, x});
    }
    void set_f32(const std::string& k, float v) {
        Value x;
        x.type = kF32;
        x.f = v;
        kv_.push_back({k, x});
    }
    void set_u64(const std::string& k, uint64_t v) {
        Value x;
        x.type = kU64;
        x.u = v;
        kv_.push_back({k, x});
    }
    void set_arr_u64(const std::string& k, const std::vector<uint64_t>& v) {
        Value x;
        x.type = kArray;
        x.arr_type = kU64;
        x.au = v;
        kv_.push_back({k, x});
    }
    void set_arr_str(const std::string& k, const std::vector<std::string>& v) {
        Value x;
        x.type = kArray;
        x.arr_type = kString;
        x.as = v;
        kv_.push_back({k, x});
    }
    // an f32 tensor; ne[0] is the contiguous extent; `data` must stay alive until write()
    void add_f32(const std::string& name, const std::vector<int64_t>& ne, const std::vector<float>& data) {
        tensors_.push_back({name, ne, data.data(), data.size()});
    }

    bool write(const std::string& path, std::string& err) const {
        std::string b;
        auto put = [&](const void* p, size_t n) { b.append(static_cast<const char*>(p), n); };
        auto put_u32 = [&](uint32_t v) { put(&v, 4); };
        auto put_u64 = [&](uint64_t v) { put(&v, 8); };
        auto put_str = [&](const std::string& s) {
            put_u64(s.size());
            put(s.data(), s.size());
        };
        put("GGUF", 4);
        put_u32(kVersion);
        put_u64(tensors_.size());
        put_u64(kv_.size());
        for (const auto& kv : kv_) {
            put_str(kv.first);
            put_u32(kv.second.type);
            switch (kv.second.type) {
                case kString: put_str(kv.second.s); break;
                case kU32: put_u32((uint32_t)kv.second.u); break;
                case kU64: put_u64(kv.second.u); break;
                case kF32: {
                    const float f = (float)kv.second.f;
                    put(&f, 4);
                    break;
                }
                case kArray:
                    put_u32(kv.second.arr_type);
                    if (kv.second.arr_type == kU64) {
                        put_u64(kv.second.au.size());
                        for (uint64_t v : kv.second.au) put_u64(v);
                    } else if (kv.second.arr_type == kString) {
                        put_u64(kv.second.as.size());
                        for (const std::string& v : kv.second.as) put_str(v);
                    } else {
                        err = "gguf writer: unsupported array type";
                        return false;
                    }
                    break;
                default: err = "gguf writer: unsupported metadata type"; return false;
            }
        }
        uint64_t off = 0;
        for (const auto& t : tensors_) {
            put_str(t.name);
            put_u32((uint32_t)t.ne.size());
            for (int64_t e : t.ne) put_u64((uint64_t)e);
            put_u32(kTensorF32);
            put_u64(off);
            off = align_up(off + t.n * 4, kDefaultAlignment);
        }
        b.resize(align_up(b.size(), kDefaultAlignment), '\0');
        // the metadata block, then every tensor's bytes and zero padding, streamed
        std::FILE* f = std::fopen(path.c_str(), "wb");
        if (!f) {
            err = "cannot open " + path + " for writing";
            return false;
        }
        static const char zeros[kDefaultAlignment] = {};
        bool ok = std::fwrite(b.data(), 1, b.size(), f) == b.size();
        for (const auto& t : tensors_) {
            if (!ok) break;
            const size_t bytes = t.n * 4, pad = (size_t)(align_up(bytes, kDefaultAlignment) - bytes);
            ok = std::fwrite(t.data, 1, bytes, f) == bytes && std::fwrite(zeros, 1, pad, f) == pad;
        }
        if (std::fclose(f) != 0 || !ok) {
            err = "failed to write " + path;
            return false;
        }
        return true;
    }

private:
    struct Tensor {
        std::string name;
        std::vector<int64_t> ne;
        const float* data;
        size_t n;
    };
    std::vector<std::pair<std::string, Value>> kv_;
    std::vector<Tensor> tensors_;
};

class Reader {
public:
    // reads and validates the whole file; false with err on anything malformed
    bool open(const std::string& path, std::string& err) {
        std::FILE* f = std::fopen(path.c_str(), "rb");
        if (!f) {
            err = "cannot open " + path;
            return false;
        }
        std::fseek(f, 0, SEEK_END);
        const long size = std::ftell(f);
        std::fseek(f, 0, SEEK_SET);
        buf_.assign(size > 0 ? (size_t)size : 0, '\0');
        const bool ok = size > 0 && std::fread(&buf_[0], 1, buf_.size(), f) == buf_.size();
        std::fclose(f);
        if (!ok) {
            err = "cannot read " + path;
            return false;
        }
        pos_ = 0;
        err_.clear();
        if (!parse()) {
            err = path + ": " + (err_.empty() ? "not a GGUF file" : err_);
            return false;
        }
        return true;
    }

    const Value* find(const std::string& key) const {
        for (const auto& kv : kv_)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
    const std::vector<TensorInfo>& tensors() const { return tensors_; }

    // a tensor's elements as f32 (f32 or f16 storage)
    bool read(const TensorInfo& t, std::vector<float>& out, std::string& err) const {
        const int64_t n = t.elements();
        const uint64_t esz = t.type == kTensorF32 ? 4 : t.type == kTensorF16 ? 2 : 0;
        if (esz == 0) {
            err = "tensor " + t.name + ": unsupported type " + std::to_string(t.type);
            return false;
        }
        // offset and n * esz must both stay inside the data section (no wrap-around)
        if (n <= 0 || data_ > buf_.size() || t.offset > buf_.size() - data_ ||
            (uint64_t)n > (buf_.size() - data_ - t.offset) / esz) {
            err = "tensor " + t.name + ": data past the end of the file";
            return false;
        }
        const uint64_t start = data_ + t.offset;
        out.resize((size_t)n);
        if (esz == 4) {
            std::memcpy(out.data(), buf_.data() + start, (size_t)n * 4);
        } else {
            for (int64_t i = 0; i < n; ++i) {
                uint16_t h;
                std::memcpy(&h, buf_.data() + start + 2 * i, 2);
                out[(size_t)i] = half_to_float(h);
            }
        }
        return true;
    }

private:
    bool need(uint64_t n) {
        if (n > buf_.size() - pos_) {
            err_ = "truncated";
            return false;
        }
        return true;
    }
    template <class T>
    bool get(T& v) {
        if (!need(sizeof(T))) return false;
        std::memcpy(&v, buf_.data() + pos_, sizeof(T));
        pos_ += sizeof(T);
        return true;
    }
    bool get_str(std::string& s) {
        uint64_t n;
        if (!get(n) || !need(n)) return false;
        s.assign(buf_.data() + pos_, (size_t)n);
        pos_ += n;
        return true;
    }
    static uint64_t scalar_size(uint32_t t) {
        switch (t) {
            case kU8: case kI8: case kBool: return 1;
            case kU16: case kI16: return 2;
            case kU32: case kI32: case kF32: return 4;
            case kU64: case kI64: case kF64: return 8;
            default: return 0;
        }
    }
    bool get_value(uint32_t type, Value& v) {
        v.type = type;
        switch (type) {
            case kString: return get_str(v.s);
            case kU8: { uint8_t x; if (!get(x)) return false; v.u = x; return true; }
            case kBool: { uint8_t x; if (!get(x)) return false; v.u = x != 0; return true; }
            case kI8: { int8_t x; if (!get(x)) return false; v.i = x; return true; }
            case kU16: { uint16_t x; if (!get(x)) return false; v.u = x; return true; }
            case kI16: { int16_t x; if (!get(x)) return false; v.i = x; return true; }
            case kU32: { uint32_t x; if (!get(x)) return false; v.u = x; return true; }
            case kI32: { int32_t x; if (!get(x)) return false; v.i = x; return true; }
            case kU64: return get(v.u);
            case kI64: return get(v.i);
            case kF32: { float x; if (!get(x)) return false; v.f = x; return true; }
            case kF64: return get(v.f);
            case kArray: {   // element type, count, elements: u64 and string arrays are kept
                uint32_t et;
                uint64_t n;
                if (!get(et) || !get(n)) return false;
                v.arr_type = et;
                if (et == kString) {
                    if (n > (buf_.size() - pos_) / 8) {   // every element needs its 8-byte length
                        err_ = "bad array";
                        return false;
                    }
                    v.as.resize((size_t)n);
                    for (uint64_t k = 0; k < n; ++k)
                        if (!get_str(v.as[(size_t)k])) return false;
                    return true;
                }
                const uint64_t es = scalar_size(et);
                if (es == 0 || n > (buf_.size() - pos_) / es) {
                    err_ = "bad array";
                    return false;
                }
                if (et == kU64) {
                    v.au.resize((size_t)n);
                    if (n) std::memcpy(v.au.data(), buf_.data() + pos_, (size_t)n * 8);
                }
                pos_ += n * es;
                return true;
            }
            default: err_ = "unknown metadata type " + std::to_string(type); return false;
        }
    }
    bool parse() {
        char magic[4];
        uint32_t version;
        uint64_t n_tensors, n_kv;
        if (!need(4)) return false;
        std::memcpy(magic, buf_.data(), 4);
        pos_ = 4;
        if (std::memcmp(magic, "GGUF", 4) != 0) {
            err_ = "not a GGUF file";
            return false;
        }
        if (!get(version) || !get(n_tensors) || !get(n_kv)) return false;
        if (version < 2 || version > 3) {
            err_ = "unsupported GGUF version " + std::to_string(version);
            return false;
        }
        uint64_t alignment = kDefaultAlignment;
        for (uint64_t k = 0; k < n_kv; ++k) {
            std::string key;
            uint32_t type;
            Value v;
            if (!get_str(key) || !get(type) || !get_value(type, v)) return false;
            if (key == "general.alignment" && type == kU32) {
                if (v.u == 0 || (v.u & (v.u - 1)) != 0) {
                    err_ = "general.alignment is not a power of two";
                    return false;
                }
                alignment = v.u;
            }
            kv_.emplace_back(key, v);
        }
        for (uint64_t k = 0; k < n_tensors; ++k) {
            TensorInfo t;
            uint32_t nd;
            if (!get_str(t.name) || !get(nd)) return false;
            if (nd > 4) {
                err_ = "tensor " + t.name + ": too many dimensions";
                return false;
            }
            t.ne.resize(nd);
            int64_t count = 1;
            for (uint32_t d = 0; d < nd; ++d) {
                uint64_t e;
                if (!get(e)) return false;
                if (e == 0 || e >= ((uint64_t)1 << 62) || __builtin_mul_overflow(count, (int64_t)e, &count)) {
                    err_ = "tensor " + t.name + ": bad extent";
                    return false;
                }
                t.ne[d] = (int64_t)e;
            }
            if (!get(t.type) || !get(t.offset)) return false;
            tensors_.push_back(t);
        }
        data_ = align_up(pos_, alignment);
        return data_ <= buf_.size();
    }

    std::string buf_, err_;
    uint64_t pos_ = 0, data_ = 0;
    std::vector<std::pair<std::string, Value>> kv_;
    std::vector<TensorInfo> tensors_;
};

}  // namespace gguf
}  // namespace sa3
