// Host Tensor (interface of the reference's src/tensor.cu:70-420).
// Differences that follow from the MI355X design:
//  * storage is reference counted and shared by views, so views stay valid
//    whatever their owner does;
//  * contiguous() is one strided-copy launch (geometry in the kernel
//    arguments) instead of a device allocation + 2 H2D copies + a stream
//    synchronize (src/tensor.cu:47-68);
//  * matmul takes transposed 2-D views as transposed GEMM operands instead
//    of materialising them.
#include <algorithm>
#include <atomic>
#include <numeric>
#include <string>

#include "../../../include/cudeep/kernels/matmul.hpp"
#include "../../../include/cudeep/memory.hpp"
#include "../../../include/cudeep/tensor.hpp"

namespace cudeep {

namespace {

std::atomic<uint64_t> g_seed{0x2545F4914F6CDD1Dull};
std::atomic<uint64_t> g_offset{0};

std::shared_ptr<void> make_storage(size_t nbytes) {
    void* p = device_malloc(nbytes);
    return std::shared_ptr<void>(p, [](void* q) {
        if (q) MemoryPool::instance().deallocate(q);
    });
}

std::string shape_str(const std::vector<int64_t>& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

}  // namespace

int cdx_dtype(DType d) {
    if (d == DType::Float32) return CDX_DTYPE_F32;
    if (d == DType::Float64) return CDX_DTYPE_F64;
    throw std::runtime_error("float16 tensors are not supported by this build");
}

Tensor::Tensor() = default;

Tensor::Tensor(const std::vector<int64_t>& shape, DType dtype) : shape_(shape), dtype_(dtype) {
    for (int64_t d : shape_) CUDEEP_ASSERT(d >= 0, "negative dimension in " + shape_str(shape_));
    compute_strides();
    const size_t n = nbytes();
    if (n > 0) {
        storage_ = make_storage(n);
        data_ = storage_.get();
    }
}

void Tensor::compute_strides() {
    strides_.assign(shape_.size(), 1);
    for (int64_t i = (int64_t)shape_.size() - 2; i >= 0; --i)
        strides_[i] = strides_[i + 1] * shape_[i + 1];
}

int64_t Tensor::numel() const {
    return std::accumulate(shape_.begin(), shape_.end(), (int64_t)1, std::multiplies<int64_t>());
}

size_t Tensor::nbytes() const { return (size_t)numel() * dtype_size(dtype_); }

bool Tensor::is_contiguous() const {
    int64_t expect = 1;
    for (int64_t i = (int64_t)shape_.size() - 1; i >= 0; --i) {
        if (shape_[i] != 1 && strides_[i] != expect) return false;
        expect *= shape_[i];
    }
    return true;
}

Tensor Tensor::zeros(const std::vector<int64_t>& shape, DType dtype) {
    Tensor t(shape, dtype);
    t.zero_();
    return t;
}

Tensor Tensor::ones(const std::vector<int64_t>& shape, DType dtype) {
    Tensor t(shape, dtype);
    t.fill_(1.0f);
    return t;
}

void Tensor::manual_seed(uint64_t seed) {
    g_seed = seed;
    g_offset = 0;
}

Tensor Tensor::randn(const std::vector<int64_t>& shape, DType dtype) {
    Tensor t(shape, dtype);
    const int64_t n = t.numel();
    const uint64_t pairs = (uint64_t)(n + 1) / 2;
    const uint64_t off = g_offset.fetch_add(pairs);
    CUDEEP_CHECK_CDX(cdx_randn(t.data_, n, cdx_dtype(dtype), g_seed.load(), off, t.stream_));
    return t;
}

Tensor Tensor::from_host(const void* host_data, const std::vector<int64_t>& shape, DType dtype) {
    Tensor t(shape, dtype);
    memcpy_h2d(t.data_, host_data, t.nbytes(), nullptr);
    return t;
}

void Tensor::to_host(void* host_dst) const {
    if (!is_contiguous()) {
        contiguous().to_host(host_dst);
        return;
    }
    if (stream_) CUDEEP_CHECK_HIP(hipStreamSynchronize(stream_));
    memcpy_d2h(host_dst, data_, nbytes(), nullptr);
}

Tensor Tensor::reshape(const std::vector<int64_t>& new_shape) const {
    std::vector<int64_t> shape = new_shape;
    int64_t known = 1, infer = -1;
    for (size_t i = 0; i < shape.size(); ++i) {
        if (shape[i] == -1) {
            CUDEEP_ASSERT(infer < 0, "reshape: only one dimension can be -1");
            infer = (int64_t)i;
        } else {
            known *= shape[i];
        }
    }
    if (infer >= 0) {
        CUDEEP_ASSERT(known > 0 && numel() % known == 0, "reshape: cannot infer dimension");
        shape[infer] = numel() / known;
    }
    int64_t n = std::accumulate(shape.begin(), shape.end(), (int64_t)1, std::multiplies<int64_t>());
    CUDEEP_ASSERT(n == numel(), "reshape: numel mismatch " + shape_str(shape_) + " -> " +
                                    shape_str(shape));
    Tensor base = is_contiguous() ? *this : contiguous();
    Tensor t = base;
    t.shape_ = shape;
    t.compute_strides();
    return t;
}

Tensor Tensor::transpose(int dim0, int dim1) const {
    const int nd = (int)shape_.size();
    if (dim0 < 0) dim0 += nd;
    if (dim1 < 0) dim1 += nd;
    CUDEEP_ASSERT(dim0 >= 0 && dim0 < nd && dim1 >= 0 && dim1 < nd, "transpose: dim out of range");
    Tensor t = *this;
    std::swap(t.shape_[dim0], t.shape_[dim1]);
    std::swap(t.strides_[dim0], t.strides_[dim1]);
    return t;
}

Tensor Tensor::contiguous() const {
    if (is_contiguous()) return *this;
    Tensor t(shape_, dtype_);
    t.stream_ = stream_;
    CUDEEP_CHECK_CDX(cdx_strided_copy(data_, t.data_, (int)shape_.size(), shape_.data(),
                                      strides_.data(), cdx_dtype(dtype_), stream_));
    return t;
}

Tensor Tensor::clone() const {
    if (!is_contiguous()) return contiguous();
    Tensor t(shape_, dtype_);
    t.stream_ = stream_;
    memcpy_d2d(t.data_, data_, nbytes(), stream_);
    return t;
}

Tensor Tensor::binary(const Tensor& other, int op, const char* name) const {
    CUDEEP_ASSERT(shape_ == other.shape_, std::string(name) + ": shape mismatch " +
                                              shape_str(shape_) + " vs " + shape_str(other.shape_));
    CUDEEP_ASSERT(dtype_ == other.dtype_, std::string(name) + ": dtype mismatch");
    Tensor a = contiguous(), b = other.contiguous();
    Tensor out(shape_, dtype_);
    out.stream_ = stream_;
    CUDEEP_CHECK_CDX(cdx_binary(op, cdx_dtype(dtype_), a.data_, b.data_, out.data_, numel(),
                                stream_));
    return out;
}

Tensor Tensor::operator+(const Tensor& o) const { return binary(o, CDX_BINARY_ADD, "add"); }
Tensor Tensor::operator-(const Tensor& o) const { return binary(o, CDX_BINARY_SUB, "sub"); }
Tensor Tensor::operator*(const Tensor& o) const { return binary(o, CDX_BINARY_MUL, "mul"); }

namespace {

// How a 2-D view enters the GEMM: as stored (row-major, leading dim ld), or
// transposed (column-major storage of the logical matrix).
struct Operand {
    Tensor t;
    bool trans;
    int64_t ld;
};

Operand as_operand(const Tensor& x) {
    const auto& s = x.shape();
    const auto& st = x.strides();
    if ((st[1] == 1 || s[1] == 1) && st[0] >= std::max<int64_t>(s[1], 1))
        return {x, false, std::max<int64_t>(st[0], 1)};
    if ((st[0] == 1 || s[0] == 1) && st[1] >= std::max<int64_t>(s[0], 1))
        return {x, true, std::max<int64_t>(st[1], 1)};
    Tensor c = x.contiguous();
    return {c, false, std::max<int64_t>(s[1], 1)};
}

}  // namespace

Tensor Tensor::matmul(const Tensor& other) const {
    CUDEEP_ASSERT(ndim() == 2 && other.ndim() == 2, "matmul: both operands must be 2-D");
    CUDEEP_ASSERT(shape_[1] == other.shape_[0], "matmul: inner dimensions differ " +
                                                    shape_str(shape_) + " x " +
                                                    shape_str(other.shape_));
    CUDEEP_ASSERT(dtype_ == other.dtype_, "matmul: dtype mismatch");
    const int64_t M = shape_[0], K = shape_[1], N = other.shape_[1];
    Tensor out({M, N}, dtype_);
    out.stream_ = stream_;
    if (M == 0 || N == 0) return out;
    if (K == 0) {
        out.zero_();
        return out;
    }
    Operand a = as_operand(*this), b = as_operand(other);
    if (dtype_ == DType::Float32) {
        kernels::launch_matmul_ex(static_cast<const float*>(a.t.data()),
                                  static_cast<const float*>(b.t.data()),
                                  static_cast<float*>(out.data_), M, N, K, a.trans, b.trans,
                                  a.ld, b.ld, N, nullptr, true, kernels::GemmEpilogue::None,
                                  stream_);
    } else if (dtype_ == DType::Float64) {
        kernels::launch_matmul_dgemm_ex(static_cast<const double*>(a.t.data()),
                                        static_cast<const double*>(b.t.data()),
                                        static_cast<double*>(out.data_), M, N, K, a.trans,
                                        b.trans, a.ld, b.ld, N, stream_);
    } else {
        throw std::runtime_error("matmul: unsupported dtype");
    }
    return out;
}

void Tensor::fill_(float value) {
    CUDEEP_ASSERT(is_contiguous(), "fill_: tensor must be contiguous");
    CUDEEP_CHECK_CDX(cdx_fill(data_, numel(), (double)value, cdx_dtype(dtype_), stream_));
}

void Tensor::zero_() { fill_(0.0f); }

}  // namespace cudeep
