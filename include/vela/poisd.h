// Drop-in replacement for the reference's src/poisd.h (emanwrxsti/vela): meow::Poisd over the C ABI
// of libvgemm.so (include/vgemm_model.h). Same names and meaning; load() returns false with the
// reference's message (src/poisd.cpp:11-54), the accessors throw std::runtime_error as
// src/poisd.cpp:56-64 do. The file is mapped, not read into memory, so there is no data() vector;
// each tensor's bytes are reachable through tensor_data(). The model hash (a SHA-256 of the file,
// src/poisd.h:28-30) belongs to the reference's consensus layer and is not provided.
#pragma once
#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../vgemm_model.h"

namespace meow {

struct PoisdTensor {
    uint8_t dtype;                 // 0 i8, 1 i16, 2 i32, 3 u8
    std::vector<uint32_t> dims;
    size_t off;                    // byte offset into the file
    size_t count;                  // element count
    size_t bytes() const {
        static const size_t SZ[4]{1, 2, 4, 1};
        return count * SZ[dtype];
    }
};

class Poisd {
public:
    Poisd() = default;
    Poisd(const Poisd&) = delete;
    Poisd& operator=(const Poisd&) = delete;
    ~Poisd() { vgemm_model_close(h_); }

    bool load(const std::string& path, std::string& error) {
        vgemm_model_close(h_);
        h_ = nullptr;
        entries_.clear();
        if (vgemm_model_open(path.c_str(), &h_) != VGEMM_OK) {
            error = vgemm_last_error();
            return false;
        }
        for (int i = 0, n = vgemm_model_count(h_); i < n; ++i) {
            const char* name = vgemm_model_name(h_, i);
            VgemmTensor t;
            if (vgemm_model_tensor(h_, name, &t) != VGEMM_OK) {
                error = vgemm_last_error();
                return false;
            }
            PoisdTensor e;
            e.dtype = uint8_t(t.dtype);
            e.dims.assign(t.dims, t.dims + (t.rank < 8 ? t.rank : 8));
            e.off = t.offset;
            e.count = t.count;
            entries_.emplace(name, std::move(e));
        }
        return true;
    }
    const std::map<std::string, PoisdTensor>& entries() const { return entries_; }
    bool has(const std::string& n) const { return entries_.count(n) != 0; }
    const PoisdTensor& get(const std::string& n) const {
        auto it = entries_.find(n);
        if (it == entries_.end()) throw std::runtime_error("missing tensor " + n);
        return it->second;
    }
    const void* tensor_data(const std::string& n) const {
        get(n);
        VgemmTensor t;
        if (vgemm_model_tensor(h_, n.c_str(), &t) != VGEMM_OK) throw std::runtime_error(vgemm_last_error());
        return t.data;
    }
    const int8_t* i8(const std::string& n) const {
        if (get(n).dtype != 0) throw std::runtime_error(n + " is not int8");
        return static_cast<const int8_t*>(tensor_data(n));
    }
    std::vector<int64_t> i32v(const std::string& n) const {   // int32 tensor widened to int64
        const PoisdTensor& e = get(n);
        if (e.dtype != 2) throw std::runtime_error(n + " is not int32");
        const uint8_t* p = static_cast<const uint8_t*>(tensor_data(n));
        std::vector<int64_t> v(e.count);
        for (size_t i = 0; i < e.count; ++i)
            v[i] = int32_t(uint32_t(p[4 * i]) | (uint32_t(p[4 * i + 1]) << 8) | (uint32_t(p[4 * i + 2]) << 16) | (uint32_t(p[4 * i + 3]) << 24));
        return v;
    }
    int64_t i32s(const std::string& n) const { return i32v(n).at(0); }
    std::string blob(const std::string& n) const {
        const PoisdTensor& e = get(n);
        return std::string(static_cast<const char*>(tensor_data(n)), e.bytes());
    }
    VgemmModel* handle() const { return h_; }

private:
    VgemmModel* h_ = nullptr;
    std::map<std::string, PoisdTensor> entries_;
};

}  // namespace meow
