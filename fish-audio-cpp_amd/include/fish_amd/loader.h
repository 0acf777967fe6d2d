// loader.h -- ModelLoader for dual_ar.bin (interface of src/model/loader.h:8-45)
// and the per-weight quantization metadata the engine derives from it
// (QuantMeta, src/engine/dual_ar_engine.h:83-88; group-size inference,
// src/engine/dual_ar_engine.cc:17-24).
#pragma once
#include "fish_amd/tensor.h"

#include <string>
#include <unordered_map>

namespace fish {

class ModelLoader {
public:
    ModelLoader() = default;
    ~ModelLoader();
    ModelLoader(const ModelLoader&) = delete;
    ModelLoader& operator=(const ModelLoader&) = delete;
    ModelLoader(ModelLoader&& other) noexcept;
    ModelLoader& operator=(ModelLoader&& other) noexcept;

    // mmap the file and parse its headers.  Returns false (and records a
    // message in last_error()) on a missing file, bad magic/version, or a
    // header table or tensor extent that runs past the end of the file.
    bool load(const std::string& bin_path);
    // Zero-copy view into the mapping; throws std::runtime_error if absent.
    TensorView get(const std::string& name) const;
    bool has(const std::string& name) const;
    size_t num_tensors() const { return order_.size(); }
    const TensorHeader& header_at(size_t i) const { return headers_.at(order_.at(i)); }
    void unload();
    const std::string& last_error() const { return err_; }
    int last_status() const { return status_; }

private:
    int fd_ = -1;
    void* mapped_data_ = nullptr;
    size_t mapped_size_ = 0;
    std::unordered_map<std::string, TensorHeader> headers_;
    std::vector<std::string> order_;
    std::string err_;
    int status_ = 0;
};

// dual_ar_engine.cc:17-24: 1-D scale or G <= 1 -> K, else ceil(K / G).
int infer_group_size_from_scale(const TensorView& weight, const TensorView& scale);

// Host-side description of one int8 weight's companions in the file
// (dual_ar_engine.cc:241-275).
struct QuantMetaHost {
    bool has_scale = false, has_smooth_inv = false, has_act_scale = false;
    int group_size = 0;
    int64_t M = 0, K = 0, groups = 0;
};
QuantMetaHost quant_meta_for(const ModelLoader& loader, const std::string& weight_name);

}  // namespace fish
