#pragma once
// Non-owning tensor descriptor for the KV-cache path.
//
// Mirrors the reference's `DataType` / `View` / `create_contiguous_view`
// (include/core/view.h:15-56) with one deliberate change: dims and strides are
// 64-bit. The reference multiplies int32 dims (view.h:30-33), which overflows
// once a paged pool passes 2^31 elements (a 120 GB FP8 pool is ~1.2e11 B).
#include <cstddef>
#include <cstdint>
#include <initializer_list>

#if defined(__HIPCC__)
#define AF_HD __host__ __device__
#else
#define AF_HD
#endif

// Same enumerators and order as the reference (view.h:15-20).
enum class DataType : int32_t {
    FP32 = 0,
    FP16 = 1,
    BF16 = 2,
    FP8_E4M3 = 3,
};

inline constexpr size_t dtype_size(DataType t) {
    return t == DataType::FP32 ? 4 : (t == DataType::FP8_E4M3 ? 1 : 2);
}

struct View {
    DataType dtype = DataType::FP16;
    void* data_ptr = nullptr;
    int64_t dims[4] = {0, 0, 0, 0};
    int64_t strides[4] = {0, 0, 0, 0};  // in elements
    int8_t num_dims = 0;

    AF_HD size_t offset(int64_t d0) const { return size_t(d0 * strides[0]); }
    AF_HD size_t offset(int64_t d0, int64_t d1) const {
        return size_t(d0 * strides[0] + d1 * strides[1]);
    }
    AF_HD size_t offset(int64_t d0, int64_t d1, int64_t d2) const {
        return size_t(d0 * strides[0] + d1 * strides[1] + d2 * strides[2]);
    }
    AF_HD size_t offset(int64_t d0, int64_t d1, int64_t d2, int64_t d3) const {
        return size_t(d0 * strides[0] + d1 * strides[1] + d2 * strides[2] + d3 * strides[3]);
    }
    template <typename T>
    AF_HD T* at_offset(size_t off) const { return static_cast<T*>(data_ptr) + off; }
    template <typename T, typename... Args>
    AF_HD T* at(Args... args) const { return at_offset<T>(offset(args...)); }

    int64_t numel() const {
        int64_t n = 1;
        for (int i = 0; i < num_dims; ++i) n *= dims[i];
        return n;
    }
};

// Row-major view over `ptr` (reference: view.h:41-56).
inline View create_contiguous_view(void* ptr, DataType type, std::initializer_list<int64_t> d) {
    View v;
    v.data_ptr = ptr;
    v.dtype = type;
    v.num_dims = static_cast<int8_t>(d.size());
    int i = 0;
    for (int64_t dim : d) v.dims[i++] = dim;
    v.strides[v.num_dims - 1] = 1;
    for (int j = v.num_dims - 2; j >= 0; --j) v.strides[j] = v.strides[j + 1] * v.dims[j + 1];
    return v;
}
