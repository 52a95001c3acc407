// Drop-in replacement for the GEMM half of the reference's device model (src/engine.h:12-37,
// src/engine.cu:11-104): meow::Lin, meow::Norm and meow::DevModel over the C ABI of libvgemm.so
// (include/vgemm_model.h). DevModel::load prepares every linear (padding to Np = 64k, Kp = 16k,
// tap-major 3x3 convolutions, wsum, the cst pack), builds the merged projections the reference
// builds (to_qkv, ff.net.0.proj.ag / agi, self_attn.qkv) and copies them, the norms' g/beta and
// the int32 tables lut.phi / lut.sigmoid to the device in one allocation owned by the Poisd.
// Differences, on purpose: a Lin carries cst only (the reference's separate int64 wsum/m/s/b
// device arrays duplicate it and no GEMM reads them), a Norm its int32 g/beta only, and mergeLins
// is part of load (the same fixed list) rather than a public call. Errors throw std::runtime_error.
#pragma once
#include <hip/hip_runtime.h>

#include <map>
#include <stdexcept>
#include <string>

#include "poisd.h"

namespace meow {

struct Lin {
    int N = 0, K = 0, Np = 0, Kp = 0;
    int8_t* w = nullptr;
    int4* cst = nullptr;   // cst[n] = {m, s, b, wsum}
    bool conv3 = false;
};

struct Norm {
    int32_t* g32 = nullptr;
    int32_t* beta32 = nullptr;
    int64_t den = 0;
    int C = 0;
};

class DevModel {
public:
    void load(int device, const Poisd& model) {
        h_ = model.handle();
        if (!h_) throw std::runtime_error("DevModel::load: model not loaded");
        if (vgemm_model_upload(h_, device) != VGEMM_OK) throw std::runtime_error(vgemm_last_error());
        this->device = device;
        bytes = vgemm_model_device_bytes(h_);
        lins_.clear();
        norms_.clear();
        for (int i = 0, n = vgemm_model_lin_count(h_); i < n; ++i) {
            const char* name = vgemm_model_lin_name(h_, i);
            VgemmLin l;
            if (vgemm_model_lin(h_, name, &l) != VGEMM_OK) throw std::runtime_error(vgemm_last_error());
            Lin L;
            L.N = l.N; L.K = l.K; L.Np = l.Np; L.Kp = l.Kp; L.conv3 = l.conv3 != 0;
            L.w = const_cast<int8_t*>(l.w);
            L.cst = reinterpret_cast<int4*>(const_cast<int32_t*>(l.cst));
            lins_[name] = L;
        }
        const int32_t* t = nullptr;
        int cnt = 0;
        if (vgemm_model_table(h_, "lut.phi", &t, &cnt) != VGEMM_OK) throw std::runtime_error(vgemm_last_error());
        lutPhi32 = const_cast<int32_t*>(t);
        if (vgemm_model_table(h_, "lut.sigmoid", &t, &cnt) != VGEMM_OK) throw std::runtime_error(vgemm_last_error());
        lutSigmoid32 = const_cast<int32_t*>(t);
    }
    const Lin& lin(const std::string& n) const {
        auto it = lins_.find(n);
        if (it == lins_.end()) throw std::runtime_error("no linear " + n);
        return it->second;
    }
    bool hasLin(const std::string& n) const { return lins_.count(n) != 0; }
    const Norm& norm(const std::string& n) const {
        auto it = norms_.find(n);
        if (it != norms_.end()) return it->second;
        VgemmNorm v;
        if (!h_ || vgemm_model_norm(h_, n.c_str(), &v) != VGEMM_OK) throw std::runtime_error("no norm " + n);
        Norm& nm = norms_[n];
        nm.g32 = const_cast<int32_t*>(v.g);
        nm.beta32 = const_cast<int32_t*>(v.beta);
        nm.den = v.den;
        nm.C = v.C;
        return nm;
    }
    int32_t* lutPhi32 = nullptr;
    int32_t* lutSigmoid32 = nullptr;
    size_t bytes = 0;
    int device = 0;

private:
    VgemmModel* h_ = nullptr;
    std::map<std::string, Lin> lins_;
    mutable std::map<std::string, Norm> norms_;
};

}  // namespace meow
