// The real-weights path (include/vgemm_model.h): POISDv1 files mapped read-only and parsed in place,
// host-side weight preparation of every linear and merged linear, and one device allocation that
// holds all prepared operands.
//
// Reference behaviour followed: src/poisd.cpp:11-54 (format, checks and messages),
// src/engine.cu:11-104 (which tensors become linears and norms, padding, the tap-major permutation of
// 3x3 convolutions, wsum, the cst pack, the merged projections). The reference reads the whole file
// into a vector, prepares each linear into its own device buffers and merges on the device; here the
// file is mapped (a 1.2 GB model is not copied), every operand is prepared on the host once --
// merged ones directly from their parts -- and a single hipMalloc receives them all, each 256-byte
// aligned, so the weights of a model sit in one contiguous region of HBM.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/vgemm_model.h"

namespace vk {
int set_error(int code, const std::string& msg);
void clear_error();
}  // namespace vk

namespace {

struct Entry {
    int dtype;
    std::vector<uint32_t> dims;
    size_t off, count, bytes;
};

struct PrepLin {
    int N = 0, K = 0, Np = 0, Kp = 0;
    bool conv3 = false;
    std::vector<int8_t> w;      // [Np x Kp]
    std::vector<int32_t> cst;   // [Np x 4]
    size_t dw = 0, dc = 0;      // device offsets
};

struct PrepNorm {
    int C = 0;
    int64_t den = 0;
    std::vector<int32_t> g, beta;
    size_t dg = 0, db = 0;
};

struct Table {
    std::vector<int32_t> v;
    size_t off = 0;
};

struct FormatError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

uint32_t rd32(const uint8_t* p) { return uint32_t(p[0]) | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16) | (uint32_t(p[3]) << 24); }

bool ends_with(const std::string& s, const char* t) {
    const size_t l = std::strlen(t);
    return s.size() >= l && s.compare(s.size() - l, l, t) == 0;
}

// the 3x3 convolutions of the UNet (src/engine.cu:14-17)
bool is_conv3x3(const std::string& base) {
    return ends_with(base, ".conv1") || ends_with(base, ".conv2") || ends_with(base, "conv_in") || ends_with(base, "conv_out") ||
           ends_with(base, "downsamplers.0.conv") || ends_with(base, "upsamplers.0.conv");
}

// tensors every model file must hold (src/poisd.cpp:47-49)
const char* const REQUIRED[] = {"unet.conv_in.w", "unet.conv_out.w", "te.tok.w", "te.pos", "lut.gauss", "lut.exp",
                                "lut.sigmoid", "lut.phi", "c.sig", "c.cin", "tok.vocab", "tok.merges"};

}  // namespace

struct VgemmModel {
    int fd = -1;
    const uint8_t* base = nullptr;
    size_t size = 0;
    std::map<std::string, Entry> entries;
    std::vector<const std::string*> names;
    bool prepared = false;
    std::map<std::string, PrepLin> lins;
    std::vector<const std::string*> lin_names;
    std::map<std::string, PrepNorm> norms;
    std::map<std::string, Table> tables;
    void* dev = nullptr;
    int device = -1;
    size_t dev_bytes = 0;

    ~VgemmModel() {
        if (dev) (void)hipFree(dev);
        if (base) munmap(const_cast<uint8_t*>(base), size);
        if (fd >= 0) close(fd);
    }

    const Entry& get(const std::string& n) const {
        auto it = entries.find(n);
        if (it == entries.end()) throw FormatError("missing tensor " + n);
        return it->second;
    }
    bool has(const std::string& n) const { return entries.count(n) != 0; }
    const int8_t* i8(const std::string& n) const {
        const Entry& e = get(n);
        if (e.dtype != VGEMM_DT_I8) throw FormatError(n + " is not int8");
        return reinterpret_cast<const int8_t*>(base + e.off);
    }
    // an int32 tensor's values (src/poisd.cpp:60-63 widens them to int64; every use narrows back)
    std::vector<int32_t> i32v(const std::string& n) const {
        const Entry& e = get(n);
        if (e.dtype != VGEMM_DT_I32) throw FormatError(n + " is not int32");
        std::vector<int32_t> v(e.count);
        for (size_t i = 0; i < e.count; ++i) v[i] = int32_t(rd32(base + e.off + 4 * i));
        return v;
    }

    void parse() {
        static const uint8_t MAGIC[8] = {'P', 'O', 'I', 'S', 'D', 'v', '1', 0};
        if (size < 12 || std::memcmp(base, MAGIC, 8) != 0) throw FormatError("bad magic (not a POISDv1 file)");
        size_t pos = 8;
        auto need = [&](size_t n) {
            if (n > size || pos > size - n) throw FormatError("truncated model file");
        };
        need(4);
        const uint32_t count = rd32(base + pos);
        pos += 4;
        for (uint32_t i = 0; i < count; ++i) {
            need(2);
            const size_t nl = size_t(base[pos]) | (size_t(base[pos + 1]) << 8);
            pos += 2;
            need(nl + 2);
            std::string name(reinterpret_cast<const char*>(base + pos), nl);
            pos += nl;
            Entry e;
            e.dtype = base[pos];
            const int nd = base[pos + 1];
            pos += 2;
            if (e.dtype > VGEMM_DT_U8) throw FormatError("bad dtype");
            need(4 * size_t(nd));
            e.count = 1;
            for (int d = 0; d < nd; ++d) {
                const uint32_t v = rd32(base + pos);
                e.dims.push_back(v);
                // a product past 2^64 cannot fit in the file either
                if (__builtin_mul_overflow(e.count, size_t(v), &e.count)) throw FormatError("truncated model file");
                pos += 4;
            }
            static const size_t SZ[4] = {1, 2, 4, 1};
            if (__builtin_mul_overflow(e.count, SZ[e.dtype], &e.bytes)) throw FormatError("truncated model file");
            need(e.bytes);
            e.off = pos;
            pos += e.bytes;
            entries.emplace(std::move(name), std::move(e));   // the first of duplicate names stays, as std::map::emplace
        }
        if (pos != size) throw FormatError("trailing data");
        for (const char* n : REQUIRED)
            if (!has(n)) throw FormatError(std::string("missing tensor ") + n);
        names.clear();
        for (const auto& kv : entries) names.push_back(&kv.first);
    }

    // one linear from "<base>.w" (src/engine.cu:19-45)
    void prepare_lin(const std::string& name, const Entry& t) {
        const std::string bs = name.substr(0, name.size() - 2);
        PrepLin L;
        L.N = int(t.dims[0]);
        L.K = int(t.dims[1]);
        L.Np = int(align_up(size_t(L.N), 64));
        L.Kp = int(align_up(size_t(L.K), 16));
        L.conv3 = is_conv3x3(bs);
        const int C = L.conv3 ? L.K / 9 : 0;
        if (L.conv3 && C * 9 != L.K) throw FormatError("conv weight K not multiple of 9: " + name);
        const std::vector<int32_t> m = i32v(bs + ".m"), s = i32v(bs + ".s"), b = i32v(bs + ".b");
        if (m.size() < size_t(L.N) || s.size() < size_t(L.N) || b.size() < size_t(L.N))
            throw FormatError("requantisation vectors of " + bs + " shorter than its " + std::to_string(L.N) + " rows");
        const int8_t* w = i8(name);
        L.w.assign(size_t(L.Np) * L.Kp, 0);
        L.cst.assign(size_t(L.Np) * 4, 0);
        for (int n = 0; n < L.Np; ++n) {
            int32_t* c = &L.cst[size_t(n) * 4];
            if (n >= L.N) {
                c[0] = 1;   // pad rows: m = 1, s = b = wsum = 0
                continue;
            }
            const int8_t* src = w + size_t(n) * L.K;
            int8_t* dst = &L.w[size_t(n) * L.Kp];
            int64_t sum = 0;
            if (L.conv3) {
                // file column c*9 + tap -> GEMM column tap*C + c
                for (int ch = 0; ch < C; ++ch)
                    for (int tap = 0; tap < 9; ++tap) dst[size_t(tap) * C + ch] = src[ch * 9 + tap];
            } else {
                std::memcpy(dst, src, size_t(L.K));
            }
            for (int k = 0; k < L.K; ++k) sum += src[k];
            c[0] = m[n];
            c[1] = s[n];
            c[2] = b[n];
            c[3] = int32_t(sum);
        }
        lins[bs] = std::move(L);
    }

    // DevModel::mergeLins (src/engine.cu:71-101): rows of the parts stacked, or alternating
    void merge(const std::string& name, const std::vector<std::string>& parts, bool interleave) {
        std::vector<const PrepLin*> ps;
        int N = 0, K = -1;
        for (const auto& pn : parts) {
            auto it = lins.find(pn);
            if (it == lins.end()) return;   // a model without these parts has no merged linear
            ps.push_back(&it->second);
            N += it->second.N;
            if (K < 0) K = it->second.K;
            else if (K != it->second.K) throw FormatError("mergeLins: K mismatch");
        }
        PrepLin L;
        L.N = N;
        L.K = K;
        L.Np = int(align_up(size_t(N), 64));
        L.Kp = ps[0]->Kp;
        L.w.assign(size_t(L.Np) * L.Kp, 0);
        L.cst.assign(size_t(L.Np) * 4, 0);
        for (int n = 0; n < L.Np; ++n) L.cst[size_t(n) * 4] = 1;
        const int P = int(ps.size());
        if (interleave) {
            const int Ni = ps[0]->N;
            for (const PrepLin* p : ps)
                if (p->N != Ni) throw FormatError("mergeLins interleave: N mismatch");
        }
        int off = 0;
        for (int i = 0; i < P; ++i) {
            const PrepLin* p = ps[i];
            for (int r = 0; r < p->N; ++r) {
                const int dst = interleave ? r * P + i : off + r;
                std::memcpy(&L.w[size_t(dst) * L.Kp], &p->w[size_t(r) * L.Kp], size_t(L.Kp));
                std::memcpy(&L.cst[size_t(dst) * 4], &p->cst[size_t(r) * 4], 16);
            }
            off += p->N;
        }
        lins[name] = std::move(L);
    }

    void prepare() {
        if (prepared) return;
        lins.clear();
        norms.clear();
        tables.clear();
        for (const auto& kv : entries) {
            const std::string& name = kv.first;
            const Entry& t = kv.second;
            if (t.dtype != VGEMM_DT_I8 || !ends_with(name, ".w") || name.size() < 2 || t.dims.size() != 2) continue;
            const std::string bs = name.substr(0, name.size() - 2);
            if (bs == "te.tok" || !has(bs + ".m")) continue;
            prepare_lin(name, t);
        }
        for (const auto& kv : entries) {
            const std::string& name = kv.first;
            if (!ends_with(name, ".g")) continue;
            const std::string bs = name.substr(0, name.size() - 2);
            if (!has(bs + ".beta") || !has(bs + ".eps")) continue;
            PrepNorm nm;
            nm.g = i32v(name);
            nm.beta = i32v(bs + ".beta");
            nm.C = int(nm.g.size());
            const std::vector<int32_t> eps = i32v(bs + ".eps");
            if (eps.empty()) throw FormatError(bs + ".eps is empty");
            nm.den = eps[0];
            norms[bs] = std::move(nm);
        }
        for (const char* n : {"lut.phi", "lut.sigmoid"}) tables[n].v = i32v(n);
        // merged projections (src/engine.cu:62-69)
        std::vector<std::string> blocks;
        for (int i = 0; i < 3; ++i)
            for (int j = 0; j < 2; ++j) blocks.push_back("unet.down_blocks." + std::to_string(i) + ".attentions." + std::to_string(j));
        blocks.push_back("unet.mid_block.attentions.0");
        for (int i = 1; i < 4; ++i)
            for (int j = 0; j < 3; ++j) blocks.push_back("unet.up_blocks." + std::to_string(i) + ".attentions." + std::to_string(j));
        for (const auto& bl : blocks) {
            const std::string b = bl + ".transformer_blocks.0";
            merge(b + ".attn1.to_qkv", {b + ".attn1.to_q", b + ".attn1.to_k", b + ".attn1.to_v"}, false);
            merge(b + ".ff.net.0.proj.ag", {b + ".ff.net.0.proj.a", b + ".ff.net.0.proj.g"}, false);
            merge(b + ".ff.net.0.proj.agi", {b + ".ff.net.0.proj.a", b + ".ff.net.0.proj.g"}, true);
        }
        for (int l = 0; l < 23; ++l) {
            const std::string p = "te.layers." + std::to_string(l);
            merge(p + ".self_attn.qkv", {p + ".self_attn.q_proj", p + ".self_attn.k_proj", p + ".self_attn.v_proj"}, false);
        }
        lin_names.clear();
        for (const auto& kv : lins) lin_names.push_back(&kv.first);
        prepared = true;
    }
};

namespace {

int format_fail(const std::exception& e) { return vk::set_error(VGEMM_ERR_FORMAT, e.what()); }

int hip_fail(hipError_t e, const char* what) { return vk::set_error(VGEMM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e)); }

}  // namespace

extern "C" {

int vgemm_model_open(const char* path, VgemmModel** out) {
    if (!out) return vk::set_error(VGEMM_ERR_ARG, "model_open: null output");
    *out = nullptr;
    if (!path) return vk::set_error(VGEMM_ERR_ARG, "model_open: null path");
    VgemmModel* m = new VgemmModel;
    m->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (m->fd < 0 || fstat(m->fd, &st) != 0) {
        delete m;
        return vk::set_error(VGEMM_ERR_FORMAT, std::string("cannot open ") + path);
    }
    m->size = size_t(st.st_size);
    if (m->size < 12) {   // too short for the magic and the count (src/poisd.cpp:22)
        delete m;
        return vk::set_error(VGEMM_ERR_FORMAT, "bad magic (not a POISDv1 file)");
    }
    void* p = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, m->fd, 0);
    if (p == MAP_FAILED) {
        m->size = 0;
        delete m;
        return vk::set_error(VGEMM_ERR_FORMAT, "read error");
    }
    m->base = static_cast<const uint8_t*>(p);
    try {
        m->parse();
    } catch (const std::exception& e) {
        delete m;
        return format_fail(e);
    }
    *out = m;
    vk::clear_error();
    return VGEMM_OK;
}

void vgemm_model_close(VgemmModel* model) { delete model; }

int vgemm_model_count(const VgemmModel* model) { return model ? int(model->names.size()) : 0; }

const char* vgemm_model_name(const VgemmModel* model, int i) {
    if (!model || i < 0 || size_t(i) >= model->names.size()) return nullptr;
    return model->names[size_t(i)]->c_str();
}

int vgemm_model_tensor(const VgemmModel* model, const char* name, VgemmTensor* out) {
    if (!model || !name || !out) return vk::set_error(VGEMM_ERR_ARG, "model_tensor: null argument");
    try {
        const Entry& e = model->get(name);
        std::memset(out, 0, sizeof *out);
        out->dtype = e.dtype;
        out->rank = int(e.dims.size());
        for (size_t d = 0; d < e.dims.size() && d < 8; ++d) out->dims[d] = e.dims[d];
        out->count = e.count;
        out->offset = e.off;
        out->bytes = e.bytes;
        out->data = model->base + e.off;
    } catch (const std::exception& e) {
        return format_fail(e);
    }
    vk::clear_error();
    return VGEMM_OK;
}

int vgemm_model_prepare(VgemmModel* model) {
    if (!model) return vk::set_error(VGEMM_ERR_ARG, "model_prepare: null model");
    try {
        model->prepare();
    } catch (const std::exception& e) {
        model->lins.clear();
        model->norms.clear();
        model->tables.clear();
        model->lin_names.clear();
        return format_fail(e);
    }
    vk::clear_error();
    return VGEMM_OK;
}

int vgemm_model_upload(VgemmModel* model, int device) {
    if (!model) return vk::set_error(VGEMM_ERR_ARG, "model_upload: null model");
    if (model->dev) return vk::set_error(VGEMM_ERR_ARG, "model_upload: already uploaded (to device " + std::to_string(model->device) + ")");
    int rc = vgemm_model_prepare(model);
    if (rc) return rc;
    // layout: every operand 256-byte aligned in one allocation
    size_t off = 0;
    auto place = [&](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes, 256);
        return o;
    };
    for (auto& kv : model->lins) {
        kv.second.dw = place(kv.second.w.size());
        kv.second.dc = place(kv.second.cst.size() * 4);
    }
    for (auto& kv : model->norms) {
        kv.second.dg = place(kv.second.g.size() * 4);
        kv.second.db = place(kv.second.beta.size() * 4);
    }
    for (auto& kv : model->tables) kv.second.off = place(kv.second.v.size() * 4);
    int prev = -1;
    hipError_t e = hipGetDevice(&prev);
    if (e != hipSuccess) return hip_fail(e, "model_upload: hipGetDevice");
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "model_upload: hipSetDevice");
    void* dev = nullptr;
    e = hipMalloc(&dev, off ? off : 256);
    auto copy = [&](size_t o, const void* src, size_t bytes) {
        if (e == hipSuccess && bytes) e = hipMemcpy(static_cast<char*>(dev) + o, src, bytes, hipMemcpyHostToDevice);
    };
    if (e == hipSuccess) {
        for (auto& kv : model->lins) {
            copy(kv.second.dw, kv.second.w.data(), kv.second.w.size());
            copy(kv.second.dc, kv.second.cst.data(), kv.second.cst.size() * 4);
        }
        for (auto& kv : model->norms) {
            copy(kv.second.dg, kv.second.g.data(), kv.second.g.size() * 4);
            copy(kv.second.db, kv.second.beta.data(), kv.second.beta.size() * 4);
        }
        for (auto& kv : model->tables) copy(kv.second.off, kv.second.v.data(), kv.second.v.size() * 4);
    }
    if (e != hipSuccess) {
        const hipError_t e0 = e;
        if (dev) (void)hipFree(dev);
        (void)hipSetDevice(prev);
        return hip_fail(e0, "model_upload");
    }
    (void)hipSetDevice(prev);
    model->dev = dev;
    model->device = device;
    model->dev_bytes = off;
    vk::clear_error();
    return VGEMM_OK;
}

size_t vgemm_model_device_bytes(const VgemmModel* model) { return model ? model->dev_bytes : 0; }

int vgemm_model_lin(const VgemmModel* model, const char* name, VgemmLin* out) {
    if (!model || !name || !out) return vk::set_error(VGEMM_ERR_ARG, "model_lin: null argument");
    if (!model->prepared) return vk::set_error(VGEMM_ERR_ARG, "model_lin: call vgemm_model_prepare first");
    auto it = model->lins.find(name);
    if (it == model->lins.end()) return vk::set_error(VGEMM_ERR_ARG, std::string("no linear ") + name);
    const PrepLin& L = it->second;
    out->N = L.N; out->K = L.K; out->Np = L.Np; out->Kp = L.Kp; out->conv3 = L.conv3 ? 1 : 0;
    out->w_host = L.w.data();
    out->cst_host = L.cst.data();
    const char* d = static_cast<const char*>(model->dev);
    out->w = d ? reinterpret_cast<const int8_t*>(d + L.dw) : nullptr;
    out->cst = d ? reinterpret_cast<const int32_t*>(d + L.dc) : nullptr;
    vk::clear_error();
    return VGEMM_OK;
}

int vgemm_model_lin_count(const VgemmModel* model) { return model ? int(model->lin_names.size()) : 0; }

const char* vgemm_model_lin_name(const VgemmModel* model, int i) {
    if (!model || i < 0 || size_t(i) >= model->lin_names.size()) return nullptr;
    return model->lin_names[size_t(i)]->c_str();
}

int vgemm_model_norm(const VgemmModel* model, const char* name, VgemmNorm* out) {
    if (!model || !name || !out) return vk::set_error(VGEMM_ERR_ARG, "model_norm: null argument");
    if (!model->prepared) return vk::set_error(VGEMM_ERR_ARG, "model_norm: call vgemm_model_prepare first");
    auto it = model->norms.find(name);
    if (it == model->norms.end()) return vk::set_error(VGEMM_ERR_ARG, std::string("no norm ") + name);
    const PrepNorm& n = it->second;
    out->C = n.C;
    out->den = n.den;
    out->g_host = n.g.data();
    out->beta_host = n.beta.data();
    const char* d = static_cast<const char*>(model->dev);
    out->g = d ? reinterpret_cast<const int32_t*>(d + n.dg) : nullptr;
    out->beta = d ? reinterpret_cast<const int32_t*>(d + n.db) : nullptr;
    vk::clear_error();
    return VGEMM_OK;
}

int vgemm_model_table(const VgemmModel* model, const char* name, const int32_t** dev, int* count) {
    if (!model || !name || !dev || !count) return vk::set_error(VGEMM_ERR_ARG, "model_table: null argument");
    auto it = model->tables.find(name);
    if (it == model->tables.end()) return vk::set_error(VGEMM_ERR_ARG, std::string("no table ") + name);
    if (!model->dev) return vk::set_error(VGEMM_ERR_ARG, "model_table: call vgemm_model_upload first");
    *dev = reinterpret_cast<const int32_t*>(static_cast<const char*>(model->dev) + it->second.off);
    *count = int(it->second.v.size());
    vk::clear_error();
    return VGEMM_OK;
}

}  // extern "C"
