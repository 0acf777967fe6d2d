// loader.cpp -- dual_ar.bin reader (ModelLoader, src/model/loader.cc:50-167)
// and its C ABI (fa_bin_*).  The file is mapped read-only; views point into
// the mapping.  Unlike the reference, the header table and every tensor's
// [offset, offset + size) are checked against the file size, so a truncated
// file fails to load instead of being read past its end.
#include "fish_amd/loader.h"
#include "../../include/fish_w8a8.h"

#include <cstring>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace fish {

ModelLoader::~ModelLoader() { unload(); }

ModelLoader::ModelLoader(ModelLoader&& o) noexcept
    : fd_(o.fd_), mapped_data_(o.mapped_data_), mapped_size_(o.mapped_size_),
      headers_(std::move(o.headers_)), order_(std::move(o.order_)) {
    o.fd_ = -1;
    o.mapped_data_ = nullptr;
    o.mapped_size_ = 0;
}

ModelLoader& ModelLoader::operator=(ModelLoader&& o) noexcept {
    if (this != &o) {
        unload();
        fd_ = o.fd_;
        mapped_data_ = o.mapped_data_;
        mapped_size_ = o.mapped_size_;
        headers_ = std::move(o.headers_);
        order_ = std::move(o.order_);
        o.fd_ = -1;
        o.mapped_data_ = nullptr;
        o.mapped_size_ = 0;
    }
    return *this;
}

void ModelLoader::unload() {
    if (mapped_data_ && mapped_size_) munmap(mapped_data_, mapped_size_);
    if (fd_ >= 0) close(fd_);
    fd_ = -1;
    mapped_data_ = nullptr;
    mapped_size_ = 0;
    headers_.clear();
    order_.clear();
}

bool ModelLoader::load(const std::string& path) {
    unload();
    auto bad = [&](int status, const std::string& msg) {
        err_ = msg;
        status_ = status;
        unload();
        return false;
    };
    fd_ = open(path.c_str(), O_RDONLY);
    if (fd_ < 0) return bad(FA_ERR_IO, "cannot open " + path);
    struct stat st;
    if (fstat(fd_, &st) < 0) return bad(FA_ERR_IO, "cannot stat " + path);
    mapped_size_ = (size_t)st.st_size;
    if (mapped_size_ < 12) return bad(FA_ERR_FORMAT, "file too small for the 12-byte header");
    mapped_data_ = mmap(nullptr, mapped_size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (mapped_data_ == MAP_FAILED) {
        mapped_data_ = nullptr;
        return bad(FA_ERR_IO, "cannot mmap " + path);
    }
    const uint8_t* base = static_cast<const uint8_t*>(mapped_data_);
    uint32_t magic, version, n;
    std::memcpy(&magic, base, 4);
    std::memcpy(&version, base + 4, 4);
    std::memcpy(&n, base + 8, 4);
    if (magic != MAGIC) return bad(FA_ERR_FORMAT, "bad magic");
    if (version != FORMAT_VERSION) return bad(FA_ERR_FORMAT, "unsupported version");
    if ((uint64_t)n * sizeof(TensorHeader) > mapped_size_ - 12)
        return bad(FA_ERR_FORMAT, "truncated header table");
    for (uint32_t i = 0; i < n; ++i) {
        TensorHeader h;
        std::memcpy(&h, base + 12 + (size_t)i * sizeof(TensorHeader), sizeof(TensorHeader));
        h.name[sizeof(h.name) - 1] = '\0';
        if (h.ndim > 8) return bad(FA_ERR_FORMAT, std::string("ndim > 8 for ") + h.name);
        if (h.data_offset > mapped_size_ || h.data_size > mapped_size_ - h.data_offset)
            return bad(FA_ERR_FORMAT, std::string("tensor data outside the file: ") + h.name);
        std::string name(h.name);
        if (!headers_.count(name)) order_.push_back(name);
        headers_[name] = h;
    }
    err_.clear();
    status_ = 0;
    return true;
}

TensorView ModelLoader::get(const std::string& name) const {
    auto it = headers_.find(name);
    if (it == headers_.end()) throw std::runtime_error("Tensor not found: " + name);
    const TensorHeader& h = it->second;
    TensorView v;
    v.data = static_cast<char*>(mapped_data_) + h.data_offset;
    v.dtype = static_cast<DType>(h.dtype_val);
    v.shape.assign(h.shape, h.shape + h.ndim);
    return v;
}

bool ModelLoader::has(const std::string& name) const { return headers_.count(name) > 0; }

int infer_group_size_from_scale(const TensorView& weight, const TensorView& scale) {
    int64_t K = 1;
    for (size_t i = 1; i < weight.shape.size(); ++i) K *= weight.shape[i];
    const int64_t groups = scale.shape.size() <= 1 ? 1 : scale.shape[1];
    return fa_infer_group_size(K, (int)scale.shape.size(), groups);
}

QuantMetaHost quant_meta_for(const ModelLoader& loader, const std::string& w) {
    QuantMetaHost m;
    TensorView wv = loader.get(w);
    m.M = wv.shape.empty() ? 1 : wv.shape[0];
    m.K = 1;
    for (size_t i = 1; i < wv.shape.size(); ++i) m.K *= wv.shape[i];
    m.has_scale = loader.has(w + "_scale");
    m.has_smooth_inv = loader.has(w + "_smooth_inv");
    m.has_act_scale = loader.has(w + "_act_scale");
    if (m.has_scale) {
        TensorView s = loader.get(w + "_scale");
        m.groups = s.shape.size() <= 1 ? 1 : s.shape[1];
        m.group_size = infer_group_size_from_scale(wv, s);
    }
    return m;
}

}  // namespace fish

struct fa_bin {
    fish::ModelLoader loader;
};

namespace fa {
void set_last_error(const std::string& msg);  // api.cpp
}

namespace {
void fill_info(const fish::TensorHeader& h, const void* base, fa_tensor_info* info) {
    std::memset(info, 0, sizeof(*info));
    std::memcpy(info->name, h.name, sizeof(info->name));
    info->dtype = h.dtype_val;
    info->ndim = h.ndim;
    for (uint32_t i = 0; i < 8; ++i) info->shape[i] = i < h.ndim ? h.shape[i] : 0;
    info->offset = h.data_offset;
    info->size = h.data_size;
    info->data = static_cast<const char*>(base) + h.data_offset;
}
}  // namespace

extern "C" {

int fa_infer_group_size(int64_t K, int scale_ndim, int64_t scale_groups) {
    if (scale_ndim <= 1 || scale_groups <= 1) return (int)K;
    return (int)((K + scale_groups - 1) / scale_groups);
}

int fa_bin_open(const char* path, fa_bin** out) {
    fa::set_last_error("");
    if (!path || !out) return FA_ERR_INVALID_ARG;
    *out = nullptr;
    fa_bin* b = new fa_bin;
    if (!b->loader.load(path)) {
        int st = b->loader.last_status();
        fa::set_last_error(b->loader.last_error());
        delete b;
        return st ? st : FA_ERR_FORMAT;
    }
    *out = b;
    return FA_OK;
}

void fa_bin_close(fa_bin* bin) { delete bin; }

int fa_bin_num_tensors(const fa_bin* bin) { return bin ? (int)bin->loader.num_tensors() : 0; }

int fa_bin_tensor_at(const fa_bin* bin, int index, fa_tensor_info* info) {
    if (!bin || !info || index < 0 || (size_t)index >= bin->loader.num_tensors())
        return FA_ERR_INVALID_ARG;
    const fish::TensorHeader& h = bin->loader.header_at((size_t)index);
    fish::TensorView v = bin->loader.get(h.name);
    fill_info(h, static_cast<const char*>(v.data) - h.data_offset, info);
    return FA_OK;
}

int fa_bin_find(const fa_bin* bin, const char* name, fa_tensor_info* info) {
    if (!bin || !name || !info) return FA_ERR_INVALID_ARG;
    if (!bin->loader.has(name)) return FA_ERR_NOT_FOUND;
    for (size_t i = 0; i < bin->loader.num_tensors(); ++i) {
        const fish::TensorHeader& h = bin->loader.header_at(i);
        if (std::strcmp(h.name, name) == 0) {
            fish::TensorView v = bin->loader.get(name);
            fill_info(h, static_cast<const char*>(v.data) - h.data_offset, info);
            return FA_OK;
        }
    }
    return FA_ERR_NOT_FOUND;
}

int fa_bin_quant_meta(const fa_bin* bin, const char* weight_name, fa_quant_meta* meta) {
    if (!bin || !weight_name || !meta) return FA_ERR_INVALID_ARG;
    if (!bin->loader.has(weight_name)) return FA_ERR_NOT_FOUND;
    fish::QuantMetaHost m = fish::quant_meta_for(bin->loader, weight_name);
    meta->has_scale = m.has_scale;
    meta->has_smooth_inv = m.has_smooth_inv;
    meta->has_act_scale = m.has_act_scale;
    meta->group_size = m.group_size;
    meta->M = m.M;
    meta->K = m.K;
    meta->groups = m.groups;
    return FA_OK;
}

int fa_bin_gate_up(const fa_bin* bin, const char* w1_name, const char* w3_name, int8_t* w13,
                   uint16_t* s13, fa_quant_meta* meta) {
    fa::set_last_error("");
    if (!bin || !w1_name || !w3_name) return FA_ERR_INVALID_ARG;
    const fish::ModelLoader& L = bin->loader;
    if (!L.has(w1_name) || !L.has(w3_name)) return FA_ERR_NOT_FOUND;
    auto fail = [](const std::string& m) {
        fa::set_last_error("fa_bin_gate_up: " + m);
        return FA_ERR_INVALID_ARG;
    };
    const std::string n1(w1_name), n3(w3_name);
    const fish::QuantMetaHost m1 = fish::quant_meta_for(L, n1), m3 = fish::quant_meta_for(L, n3);
    const fish::TensorView v1 = L.get(n1), v3 = L.get(n3);
    if (v1.dtype != fish::DType::INT8 || v3.dtype != fish::DType::INT8 || !m1.has_scale ||
        !m3.has_scale)
        return fail("w1 and w3 must be int8 weights with fp16 scales");
    if (m1.M != m3.M || m1.K != m3.K || m1.groups != m3.groups || m1.group_size != m3.group_size)
        return fail("w1 and w3 differ in shape or group size");
    // one input quantization feeds both halves: their smooth_inv and static
    // act_scale companions must agree (absent in both, or byte-identical)
    for (const char* sfx : {"_smooth_inv", "_act_scale"}) {
        const bool h1 = L.has(n1 + sfx), h3 = L.has(n3 + sfx);
        if (h1 != h3) return fail(std::string("only one of w1 / w3 has ") + (sfx + 1));
        if (h1) {
            const fish::TensorView a = L.get(n1 + sfx), c = L.get(n3 + sfx);
            const size_t na = (size_t)a.numel() * 2, nc = (size_t)c.numel() * 2;
            if (na != nc || std::memcmp(a.data, c.data, na) != 0)
                return fail(std::string("w1 and w3 ") + (sfx + 1) +
                            " differ: their inputs quantize differently");
        }
    }
    const fish::TensorView sv1 = L.get(n1 + "_scale"), sv3 = L.get(n3 + "_scale");
    if (sv1.dtype != fish::DType::FP16 || sv3.dtype != fish::DType::FP16 ||
        sv1.numel() != m1.M * m1.groups || sv3.numel() != sv1.numel())
        return fail("scale tensors are not fp16 [M] / [M, G]");
    if (meta) {
        meta->has_scale = 1;
        meta->has_smooth_inv = m1.has_smooth_inv;
        meta->has_act_scale = m1.has_act_scale;
        meta->group_size = m1.group_size;
        meta->M = 2 * m1.M;
        meta->K = m1.K;
        meta->groups = m1.groups;
    }
    const size_t K = (size_t)m1.K, G = (size_t)m1.groups;
    const int8_t* a = static_cast<const int8_t*>(v1.data);
    const int8_t* c = static_cast<const int8_t*>(v3.data);
    const uint16_t* sa = static_cast<const uint16_t*>(sv1.data);
    const uint16_t* sc = static_cast<const uint16_t*>(sv3.data);
    for (int64_t i = 0; i < m1.M; ++i) {
        if (w13) {
            std::memcpy(w13 + (2 * i) * K, a + i * K, K);
            std::memcpy(w13 + (2 * i + 1) * K, c + i * K, K);
        }
        if (s13) {
            std::memcpy(s13 + (2 * i) * G, sa + i * G, G * 2);
            std::memcpy(s13 + (2 * i + 1) * G, sc + i * G, G * 2);
        }
    }
    return FA_OK;
}

}  // extern "C"
