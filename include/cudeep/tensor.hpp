// Host Tensor of the C++ API: owning or view, shape + strides, dtype, and
// the stream its work is enqueued on -- the interface of the reference's
// cudeep::Tensor (include/cudeep/tensor.cuh:13-67).  Storage comes from
// MemoryPool and is shared between a tensor and its views (reference
// counted), so a view never outlives its data.  matmul accepts transposed
// 2-D views directly (the GEMM reads them with a transposed operand), so
// x.matmul(w.transpose(0, 1)) makes no copy.
#pragma once

#include <memory>
#include <vector>

#include "common.hpp"
#include "error.hpp"

namespace cudeep {

class Tensor {
public:
    Tensor();
    Tensor(const std::vector<int64_t>& shape, DType dtype = DType::Float32);
    ~Tensor() = default;

    Tensor(const Tensor& other) = default;             // shares storage
    Tensor(Tensor&& other) noexcept = default;
    Tensor& operator=(const Tensor& other) = default;
    Tensor& operator=(Tensor&& other) noexcept = default;

    void* data() const { return data_; }
    const std::vector<int64_t>& shape() const { return shape_; }
    const std::vector<int64_t>& strides() const { return strides_; }
    int64_t ndim() const { return static_cast<int64_t>(shape_.size()); }
    int64_t numel() const;
    size_t nbytes() const;
    DType dtype() const { return dtype_; }

    static Tensor zeros(const std::vector<int64_t>& shape, DType dtype = DType::Float32);
    static Tensor ones(const std::vector<int64_t>& shape, DType dtype = DType::Float32);
    static Tensor randn(const std::vector<int64_t>& shape, DType dtype = DType::Float32);
    static Tensor from_host(const void* host_data, const std::vector<int64_t>& shape,
                            DType dtype = DType::Float32);
    // Seed of the randn stream (each randn call draws a fresh range).
    static void manual_seed(uint64_t seed);

    void to_host(void* host_dst) const;
    Tensor reshape(const std::vector<int64_t>& new_shape) const;
    Tensor transpose(int dim0, int dim1) const;
    Tensor contiguous() const;
    bool is_contiguous() const;
    Tensor clone() const;                              // deep copy, contiguous

    Tensor operator+(const Tensor& other) const;
    Tensor operator-(const Tensor& other) const;
    Tensor operator*(const Tensor& other) const;

    Tensor matmul(const Tensor& other) const;

    void fill_(float value);
    void zero_();

    hipStream_t stream() const { return stream_; }
    void set_stream(hipStream_t stream) { stream_ = stream; }

private:
    void compute_strides();
    Tensor binary(const Tensor& other, int op, const char* name) const;

    std::shared_ptr<void> storage_;
    void* data_ = nullptr;
    std::vector<int64_t> shape_;
    std::vector<int64_t> strides_;
    DType dtype_ = DType::Float32;
    hipStream_t stream_ = nullptr;
};

// cdx dtype code of a tensor (float32 / float64 only).
int cdx_dtype(DType d);

}  // namespace cudeep
