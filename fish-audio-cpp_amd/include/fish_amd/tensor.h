// tensor.h -- the dual_ar.bin container types (src/model/tensor.h:8-67).
// The on-disk layout has to be byte-identical to the reference's, so the enum
// values, the 344-byte header record and the magic/version are the same.
#pragma once
#include <cstdint>
#include <stdexcept>
#include <vector>

namespace fish {

enum class DType : uint32_t { FP32 = 0, FP16 = 1, BF16 = 2, INT8 = 3 };

constexpr int64_t dtype_size(DType dt) {
    return dt == DType::FP32 ? 4 : dt == DType::INT8 ? 1 : 2;
}

// Non-owning view into tensor data (host mapping or device buffer).
struct TensorView {
    void* data = nullptr;
    DType dtype = DType::FP16;
    std::vector<int64_t> shape;

    template <typename T> T* as() { return static_cast<T*>(data); }
    template <typename T> const T* as() const { return static_cast<const T*>(data); }

    int64_t numel() const {
        int64_t n = 1;
        for (int64_t s : shape) {
            if (s < 0 || (s != 0 && n > INT64_MAX / s)) throw std::overflow_error("TensorView::numel overflow");
            n *= s;
        }
        return n;
    }
    int64_t nbytes() const { return numel() * dtype_size(dtype); }
};

// One header record of the .bin file: name[256], dtype, ndim, shape[8],
// data offset (256-byte aligned), data size; 344 bytes with alignment padding.
struct TensorHeader {
    char name[256];
    uint32_t dtype_val;
    uint32_t ndim;
    int64_t shape[8];
    uint64_t data_offset;
    uint64_t data_size;
};
static_assert(sizeof(TensorHeader) == 344, "TensorHeader must be 344 bytes");

inline constexpr uint32_t MAGIC = 0x46495348;  // "FISH"
inline constexpr uint32_t FORMAT_VERSION = 1;

}  // namespace fish
