// pybind11 module `_cudeep_core`: the Python surface of the reference's
// src/bindings/module.cpp:75-981, restricted to the dense-contraction path
// (Tensor + matmul, conv2d forward / backward, broadcast_add,
// sum_reduce_rows, sum, relu / gelu / sigmoid / silu / activation_backward, Stream / Event /
// MemoryPool, device_info), with the same names, argument names and
// defaults, plus the entry points this build adds: linear_forward (one
// fused GEMM for x W^T + b with an activation), linear_weight_grad /
// linear_input_grad (a Linear layer's backward GEMMs with the bias gradient
// and the producer's activation derivative in their epilogues), matmul_ex
// (transposed operands), conv2d_backward_bias (GPU bias gradient) and the
// matmul precision switch.  Errors surface as RuntimeError (std::runtime_error).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <string>

#include "../../../include/cudeep/kernels/activation.hpp"
#include "../../../include/cudeep/kernels/conv.hpp"
#include "../../../include/cudeep/kernels/elementwise.hpp"
#include "../../../include/cudeep/kernels/matmul.hpp"
#include "../../../include/cudeep/kernels/reduce.hpp"
#include "../../../include/cudeep/kernels/unary.hpp"
#include "../../../include/cudeep/memory.hpp"
#include "../../../include/cudeep/stream.hpp"
#include "../../../include/cudeep/tensor.hpp"

namespace py = pybind11;
using namespace cudeep;

namespace {

// Unlike the reference (module.cpp:26-28), a contiguous tensor is used as
// is; only a strided view is copied.
inline Tensor ensure_contiguous(const Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }

void require_f32(const Tensor& t, const char* fn) {
    if (t.dtype() != DType::Float32)
        throw std::runtime_error(std::string(fn) + ": only float32 is supported by this build");
}

kernels::ActivationType parse_act(const std::string& name) {
    if (name == "relu") return kernels::ActivationType::ReLU;
    if (name == "gelu") return kernels::ActivationType::GELU;
    if (name == "silu") return kernels::ActivationType::SiLU;
    if (name == "sigmoid") return kernels::ActivationType::Sigmoid;
    if (name == "tanh") return kernels::ActivationType::Tanh;
    if (name == "leaky_relu") return kernels::ActivationType::LeakyReLU;
    throw std::runtime_error("Unknown activation: " + name);
}

void require_f32_or_f64(const Tensor& t, const char* fn) {
    if (t.dtype() != DType::Float32 && t.dtype() != DType::Float64)
        throw std::runtime_error(std::string(fn) + ": float32 or float64 required");
}

Tensor activation(const Tensor& t, kernels::ActivationType act, float alpha = 0.01f) {
    Tensor in = ensure_contiguous(t);
    require_f32_or_f64(in, "activation");
    Tensor out(in.shape(), in.dtype());
    if (in.dtype() == DType::Float64)
        kernels::launch_activation_forward_kernel<double>(static_cast<const double*>(in.data()),
                                                          static_cast<double*>(out.data()),
                                                          in.numel(), act, alpha, in.stream());
    else
        kernels::launch_activation_forward_kernel<float>(static_cast<const float*>(in.data()),
                                                         static_cast<float*>(out.data()),
                                                         in.numel(), act, alpha, in.stream());
    return out;
}

struct ConvGeom {
    int B, IC, IH, IW, OC, KH, KW, SH, SW, PH, PW, OH, OW;
};

ConvGeom conv_geom(const std::vector<int64_t>& ishape, const std::vector<int64_t>& wshape,
                   const std::vector<int>& stride, const std::vector<int>& padding) {
    if (ishape.size() != 4 || wshape.size() != 4)
        throw std::runtime_error("conv2d: input must be NCHW and weight OIHW (4-D)");
    if (stride.size() != 2 || padding.size() != 2)
        throw std::runtime_error("conv2d: stride and padding must have 2 entries");
    ConvGeom g;
    g.B = (int)ishape[0]; g.IC = (int)ishape[1]; g.IH = (int)ishape[2]; g.IW = (int)ishape[3];
    g.OC = (int)wshape[0]; g.KH = (int)wshape[2]; g.KW = (int)wshape[3];
    g.SH = stride[0]; g.SW = stride[1]; g.PH = padding[0]; g.PW = padding[1];
    if (wshape[1] != ishape[1]) throw std::runtime_error("conv2d: channel mismatch");
    if (g.SH <= 0 || g.SW <= 0 || g.PH < 0 || g.PW < 0)
        throw std::runtime_error("conv2d: stride must be positive and padding non-negative");
    if (g.IH + 2 * g.PH < g.KH || g.IW + 2 * g.PW < g.KW)
        throw std::runtime_error("conv2d: kernel larger than padded input");
    g.OH = (g.IH + 2 * g.PH - g.KH) / g.SH + 1;
    g.OW = (g.IW + 2 * g.PW - g.KW) / g.SW + 1;
    return g;
}

kernels::GemmEpilogue parse_epi(const std::string& a) {
    if (a == "none" || a.empty()) return kernels::GemmEpilogue::None;
    if (a == "relu") return kernels::GemmEpilogue::ReLU;
    if (a == "gelu") return kernels::GemmEpilogue::GELU;
    if (a == "silu") return kernels::GemmEpilogue::SiLU;
    if (a == "sigmoid") return kernels::GemmEpilogue::Sigmoid;
    throw std::runtime_error("linear_forward: activation must be none, relu, gelu, silu or sigmoid");
}

int64_t leading_dim(const Tensor& t) {
    return t.shape()[1] > 1 ? t.shape()[1] : 1;
}

}  // namespace

PYBIND11_MODULE(_cudeep_core, m) {
    m.doc() = "cuDeep dense-contraction path on MI355X (gfx950)";

    py::enum_<DType>(m, "DType")
        .value("float16", DType::Float16)
        .value("float32", DType::Float32)
        .value("float64", DType::Float64);

    py::enum_<Layout>(m, "Layout").value("NCHW", Layout::NCHW).value("NHWC", Layout::NHWC);

    py::class_<Tensor>(m, "Tensor")
        .def(py::init<const std::vector<int64_t>&, DType>(), py::arg("shape"),
             py::arg("dtype") = DType::Float32)
        .def("shape", &Tensor::shape)
        .def("strides", &Tensor::strides)
        .def("ndim", &Tensor::ndim)
        .def("numel", &Tensor::numel)
        .def("nbytes", &Tensor::nbytes)
        .def("dtype", &Tensor::dtype)
        .def("is_contiguous", &Tensor::is_contiguous)
        .def("reshape", &Tensor::reshape)
        .def("transpose", &Tensor::transpose, py::arg("dim0"), py::arg("dim1"))
        .def("contiguous", &Tensor::contiguous)
        .def("clone", &Tensor::clone)
        .def("fill_", &Tensor::fill_)
        .def("zero_", &Tensor::zero_)
        .def("matmul", &Tensor::matmul)
        .def("__add__", &Tensor::operator+)
        .def("__sub__", &Tensor::operator-)
        .def("__mul__", &Tensor::operator*)
        .def("data_ptr", [](const Tensor& t) { return reinterpret_cast<uintptr_t>(t.data()); })
        .def_static("zeros", &Tensor::zeros, py::arg("shape"), py::arg("dtype") = DType::Float32)
        .def_static("ones", &Tensor::ones, py::arg("shape"), py::arg("dtype") = DType::Float32)
        .def_static("randn", &Tensor::randn, py::arg("shape"), py::arg("dtype") = DType::Float32)
        .def_static("manual_seed", &Tensor::manual_seed, py::arg("seed"))
        .def("numpy", [](const Tensor& t) -> py::object {
            std::vector<ssize_t> shp(t.shape().begin(), t.shape().end());
            if (t.dtype() == DType::Float32) {
                py::array_t<float> r(shp);
                t.to_host(r.mutable_data());
                return std::move(r);
            }
            if (t.dtype() == DType::Float64) {
                py::array_t<double> r(shp);
                t.to_host(r.mutable_data());
                return std::move(r);
            }
            throw std::runtime_error("numpy() unsupported for this dtype");
        })
        .def_static("from_numpy", [](py::array arr) {
            std::vector<int64_t> shape(arr.shape(), arr.shape() + arr.ndim());
            if (py::isinstance<py::array_t<float>>(arr) &&
                arr.dtype().equal(py::dtype::of<float>())) {
                auto c = py::array_t<float, py::array::c_style | py::array::forcecast>::ensure(arr);
                return Tensor::from_host(c.data(), shape, DType::Float32);
            }
            if (arr.dtype().equal(py::dtype::of<double>())) {
                auto c = py::array_t<double, py::array::c_style | py::array::forcecast>::ensure(arr);
                return Tensor::from_host(c.data(), shape, DType::Float64);
            }
            throw std::runtime_error("Unsupported numpy dtype");
        })
        .def("__repr__", [](const Tensor& t) {
            std::string s = "cuDeep.Tensor(shape=[";
            for (size_t i = 0; i < t.shape().size(); ++i)
                s += (i ? ", " : "") + std::to_string(t.shape()[i]);
            s += "], dtype=";
            s += t.dtype() == DType::Float64 ? "float64" : t.dtype() == DType::Float32 ? "float32"
                                                                                       : "float16";
            return s + ")";
        });

    py::class_<Stream>(m, "Stream").def(py::init<>()).def("synchronize", &Stream::synchronize);

    py::class_<Event>(m, "Event")
        .def(py::init<>())
        .def("record", [](Event& e) { e.record(nullptr); })
        .def("record", [](Event& e, Stream& s) { e.record(s.get()); }, py::arg("stream"))
        .def("synchronize", &Event::synchronize)
        .def("elapsed_ms", &Event::elapsed_ms);

    py::class_<MemoryPool, std::unique_ptr<MemoryPool, py::nodelete>>(m, "MemoryPool")
        .def_static("instance", &MemoryPool::instance, py::return_value_policy::reference)
        .def("release_cached", &MemoryPool::release_cached)
        .def_property_readonly("allocated_bytes", &MemoryPool::allocated_bytes)
        .def_property_readonly("cached_bytes", &MemoryPool::cached_bytes);

    // ---- activations ----
    m.def("relu", [](const Tensor& t) { return activation(t, kernels::ActivationType::ReLU); },
          py::arg("input"));
    m.def("gelu", [](const Tensor& t) { return activation(t, kernels::ActivationType::GELU); },
          py::arg("input"));
    m.def("sigmoid", [](const Tensor& t) { return activation(t, kernels::ActivationType::Sigmoid); },
          py::arg("input"));
    m.def("silu", [](const Tensor& t) { return activation(t, kernels::ActivationType::SiLU); },
          py::arg("input"));
    m.def("tanh_act", [](const Tensor& t) { return activation(t, kernels::ActivationType::Tanh); },
          py::arg("input"));
    m.def("leaky_relu",
          [](const Tensor& t, float alpha) {
              return activation(t, kernels::ActivationType::LeakyReLU, alpha);
          },
          py::arg("input"), py::arg("alpha") = 0.01f);
    m.def("activation_backward",
          [](const Tensor& grad_output, const Tensor& input, const std::string& act_name,
             float alpha) {
              Tensor go = ensure_contiguous(grad_output), in = ensure_contiguous(input);
              require_f32_or_f64(in, "activation_backward");
              if (go.shape() != in.shape() || go.dtype() != in.dtype())
                  throw std::runtime_error("activation_backward: shape / dtype mismatch");
              Tensor gi(in.shape(), in.dtype());
              if (in.dtype() == DType::Float64)
                  kernels::launch_activation_backward_kernel<double>(
                      static_cast<const double*>(go.data()), static_cast<const double*>(in.data()),
                      static_cast<double*>(gi.data()), in.numel(), parse_act(act_name), alpha,
                      in.stream());
              else
                  kernels::launch_activation_backward_kernel<float>(
                      static_cast<const float*>(go.data()), static_cast<const float*>(in.data()),
                      static_cast<float*>(gi.data()), in.numel(), parse_act(act_name), alpha,
                      in.stream());
              return gi;
          },
          py::arg("grad_output"), py::arg("input"), py::arg("act_name"), py::arg("alpha") = 0.01f);

    // ---- reductions / broadcast ----
    m.def("sum", [](const Tensor& t) {
        Tensor in = ensure_contiguous(t);
        require_f32_or_f64(in, "sum");
        Tensor out({1}, in.dtype());
        if (in.dtype() == DType::Float32)
            kernels::launch_sum_kernel<float>(static_cast<const float*>(in.data()),
                                              static_cast<float*>(out.data()), in.numel(),
                                              in.stream());
        else
            kernels::launch_sum_kernel<double>(static_cast<const double*>(in.data()),
                                               static_cast<double*>(out.data()), in.numel(),
                                               in.stream());
        return out;
    }, py::arg("input"));

    m.def("broadcast_add", [](const Tensor& matrix, const Tensor& row) {
        Tensor mat = ensure_contiguous(matrix), r = ensure_contiguous(row);
        const auto& ms = mat.shape();
        const auto& rs = r.shape();
        if (ms.size() != 2 || rs.size() != 1 || ms[1] != rs[0])
            throw std::runtime_error(
                "broadcast_add: requires matrix [N,M] and row [M], got incompatible shapes");
        require_f32_or_f64(mat, "broadcast_add");
        if (mat.dtype() != r.dtype()) throw std::runtime_error("broadcast_add: dtype mismatch");
        Tensor out(ms, mat.dtype());
        if (mat.dtype() == DType::Float64)
            kernels::launch_broadcast_add_row_kernel<double>(
                static_cast<const double*>(mat.data()), static_cast<const double*>(r.data()),
                static_cast<double*>(out.data()), ms[0], ms[1], mat.stream());
        else
            kernels::launch_broadcast_add_row_kernel<float>(
                static_cast<const float*>(mat.data()), static_cast<const float*>(r.data()),
                static_cast<float*>(out.data()), ms[0], ms[1], mat.stream());
        return out;
    }, py::arg("matrix"), py::arg("row"));

    m.def("sum_reduce_rows", [](const Tensor& t) {
        Tensor in = ensure_contiguous(t);
        if (in.ndim() != 2) throw std::runtime_error("sum_reduce_rows: input must be 2-D");
        require_f32_or_f64(in, "sum_reduce_rows");
        Tensor out({in.shape()[1]}, in.dtype());
        if (in.dtype() == DType::Float64)
            kernels::launch_sum_reduce_rows_kernel<double>(static_cast<const double*>(in.data()),
                                                           static_cast<double*>(out.data()),
                                                           in.shape()[0], in.shape()[1],
                                                           in.stream());
        else
            kernels::launch_sum_reduce_rows_kernel<float>(static_cast<const float*>(in.data()),
                                                          static_cast<float*>(out.data()),
                                                          in.shape()[0], in.shape()[1],
                                                          in.stream());
        return out;
    }, py::arg("input"));

    // ---- GEMM entry points added by this build ----
    m.def("matmul_ex",
          [](const Tensor& a, const Tensor& b, bool trans_a, bool trans_b) {
              Tensor A = ensure_contiguous(a), B = ensure_contiguous(b);
              if (A.ndim() != 2 || B.ndim() != 2)
                  throw std::runtime_error("matmul_ex: operands must be 2-D");
              require_f32_or_f64(A, "matmul_ex");
              require_f32_or_f64(B, "matmul_ex");
              if (A.dtype() != B.dtype()) throw std::runtime_error("matmul_ex: dtype mismatch");
              const int64_t M = trans_a ? A.shape()[1] : A.shape()[0];
              const int64_t K = trans_a ? A.shape()[0] : A.shape()[1];
              const int64_t K2 = trans_b ? B.shape()[1] : B.shape()[0];
              const int64_t N = trans_b ? B.shape()[0] : B.shape()[1];
              if (K != K2) throw std::runtime_error("matmul_ex: inner dimensions differ");
              Tensor out({M, N}, A.dtype());
              if (M * N == 0) return out;
              if (A.dtype() == DType::Float64)
                  kernels::launch_matmul_dgemm_ex(
                      static_cast<const double*>(A.data()), static_cast<const double*>(B.data()),
                      static_cast<double*>(out.data()), M, N, K, trans_a, trans_b, leading_dim(A),
                      leading_dim(B), N, A.stream());
              else
                  kernels::launch_matmul_ex(
                      static_cast<const float*>(A.data()), static_cast<const float*>(B.data()),
                      static_cast<float*>(out.data()), M, N, K, trans_a, trans_b, leading_dim(A),
                      leading_dim(B), N, nullptr, true, kernels::GemmEpilogue::None, A.stream());
              return out;
          },
          py::arg("a"), py::arg("b"), py::arg("trans_a") = false, py::arg("trans_b") = false);

    m.def("linear_weight_grad",
          [](const Tensor& dz, const Tensor& x, bool with_bias) {
              Tensor Z = ensure_contiguous(dz), X = ensure_contiguous(x);
              if (Z.ndim() != 2 || X.ndim() != 2 || Z.shape()[0] != X.shape()[0])
                  throw std::runtime_error(
                      "linear_weight_grad: dz [N, out] and x [N, in] required");
              require_f32(Z, "linear_weight_grad");
              require_f32(X, "linear_weight_grad");
              const int64_t batch = Z.shape()[0], out_f = Z.shape()[1], in_f = X.shape()[1];
              Tensor gw({out_f, in_f}, DType::Float32);
              Tensor gb({out_f}, DType::Float32);
              if (out_f > 0)
                  kernels::launch_linear_weight_grad(
                      static_cast<const float*>(Z.data()), static_cast<const float*>(X.data()),
                      static_cast<float*>(gw.data()),
                      with_bias ? static_cast<float*>(gb.data()) : nullptr, batch, out_f, in_f,
                      Z.stream());
              return py::make_tuple(gw, with_bias ? py::cast(gb) : py::none());
          },
          py::arg("dz"), py::arg("x"), py::arg("with_bias") = true);

    m.def("linear_input_grad",
          [](const Tensor& dz, const Tensor& weight, py::object aux_obj,
             const std::string& activation) {
              Tensor Z = ensure_contiguous(dz), W = ensure_contiguous(weight);
              if (Z.ndim() != 2 || W.ndim() != 2 || Z.shape()[1] != W.shape()[0])
                  throw std::runtime_error(
                      "linear_input_grad: dz [N, out] and weight [out, in] required");
              require_f32(Z, "linear_input_grad");
              require_f32(W, "linear_input_grad");
              const kernels::GemmEpilogue act = parse_epi(activation);
              const int64_t batch = Z.shape()[0], out_f = Z.shape()[1], in_f = W.shape()[1];
              Tensor A;
              const float* aptr = nullptr;
              if (act != kernels::GemmEpilogue::None) {
                  if (aux_obj.is_none())
                      throw std::runtime_error("linear_input_grad: an activation needs aux");
                  A = ensure_contiguous(aux_obj.cast<Tensor>());
                  require_f32(A, "linear_input_grad");
                  if (A.ndim() != 2 || A.shape()[0] != batch || A.shape()[1] != in_f)
                      throw std::runtime_error("linear_input_grad: aux must be [N, in]");
                  aptr = static_cast<const float*>(A.data());
              }
              Tensor gx({batch, in_f}, DType::Float32);
              if (batch * in_f == 0) return gx;
              kernels::launch_linear_input_grad(
                  static_cast<const float*>(Z.data()), static_cast<const float*>(W.data()), aptr,
                  static_cast<float*>(gx.data()), batch, out_f, in_f, act, Z.stream());
              return gx;
          },
          py::arg("dz"), py::arg("weight"), py::arg("aux") = py::none(),
          py::arg("activation") = "none");

    m.def("linear_forward",
          [](const Tensor& x, const Tensor& weight, py::object bias_obj,
             const std::string& activation) {
              Tensor X = ensure_contiguous(x), W = ensure_contiguous(weight);
              if (X.ndim() != 2 || W.ndim() != 2 || X.shape()[1] != W.shape()[1])
                  throw std::runtime_error("linear_forward: x [N, in] and weight [out, in] required");
              require_f32(X, "linear_forward");
              require_f32(W, "linear_forward");
              Tensor b;
              const float* bptr = nullptr;
              if (!bias_obj.is_none()) {
                  b = ensure_contiguous(bias_obj.cast<Tensor>());
                  require_f32(b, "linear_forward");
                  if (b.numel() != W.shape()[0])
                      throw std::runtime_error("linear_forward: bias must have out_features entries");
                  bptr = static_cast<const float*>(b.data());
              }
              const int64_t M = X.shape()[0], K = X.shape()[1], N = W.shape()[0];
              Tensor out({M, N}, DType::Float32);
              if (M * N == 0) return out;
              kernels::launch_matmul_ex(static_cast<const float*>(X.data()),
                                        static_cast<const float*>(W.data()),
                                        static_cast<float*>(out.data()), M, N, K, false, true,
                                        K > 1 ? K : 1, K > 1 ? K : 1, N, bptr, true,
                                        parse_epi(activation), X.stream());
              return out;
          },
          py::arg("x"), py::arg("weight"), py::arg("bias") = py::none(),
          py::arg("activation") = "none");

    m.def("set_matmul_precision", [](const std::string& p) {
        if (p == "fp32") kernels::set_matmul_precision(kernels::MatmulPrecision::FP32);
        else if (p == "tf32") kernels::set_matmul_precision(kernels::MatmulPrecision::TF32Mode);
        else if (p == "tf32x4") kernels::set_matmul_precision(kernels::MatmulPrecision::TF32Mode4);
        else throw std::runtime_error("set_matmul_precision: 'fp32', 'tf32' or 'tf32x4'");
    }, py::arg("precision"));
    m.def("get_matmul_precision", []() {
        const auto p = kernels::get_matmul_precision();
        return p == kernels::MatmulPrecision::FP32        ? "fp32"
               : p == kernels::MatmulPrecision::TF32Mode4 ? "tf32x4"
                                                          : "tf32";
    });

    m.def("set_conv_algorithm", [](const std::string& a) {
        if (a == "auto") kernels::set_conv_algorithm(kernels::ConvAlgorithm::Auto);
        else if (a == "im2col") kernels::set_conv_algorithm(kernels::ConvAlgorithm::Im2col);
        else if (a == "winograd") kernels::set_conv_algorithm(kernels::ConvAlgorithm::Winograd);
        else if (a == "implicit") kernels::set_conv_algorithm(kernels::ConvAlgorithm::Implicit);
        else throw std::runtime_error("set_conv_algorithm: 'auto', 'im2col', 'winograd' or 'implicit'");
    }, py::arg("algorithm"));
    m.def("get_conv_algorithm", []() {
        const auto a = kernels::get_conv_algorithm();
        return a == kernels::ConvAlgorithm::Im2col     ? "im2col"
               : a == kernels::ConvAlgorithm::Winograd ? "winograd"
               : a == kernels::ConvAlgorithm::Implicit ? "implicit"
                                                       : "auto";
    });

    // ---- conv ----
    m.def("conv2d_forward",
          [](const Tensor& input, const Tensor& weight, py::object bias_obj,
             std::vector<int> stride, std::vector<int> padding) {
              Tensor in = ensure_contiguous(input), w = ensure_contiguous(weight);
              require_f32_or_f64(in, "conv2d_forward");
              if (w.dtype() != in.dtype())
                  throw std::runtime_error("conv2d_forward: input and weight dtypes differ");
              ConvGeom g = conv_geom(in.shape(), w.shape(), stride, padding);
              Tensor out({g.B, g.OC, g.OH, g.OW}, in.dtype());
              Tensor b;
              const void* bptr = nullptr;
              if (!bias_obj.is_none()) {
                  b = ensure_contiguous(bias_obj.cast<Tensor>());
                  if (b.numel() != g.OC) throw std::runtime_error("conv2d_forward: bias size");
                  if (b.dtype() != in.dtype())
                      throw std::runtime_error("conv2d_forward: bias dtype differs");
                  bptr = b.data();
              }
              if (in.dtype() == DType::Float64)
                  kernels::launch_conv2d_forward_kernel<double>(
                      static_cast<const double*>(in.data()), static_cast<const double*>(w.data()),
                      static_cast<const double*>(bptr), static_cast<double*>(out.data()), g.B,
                      g.IC, g.OC, g.IH, g.IW, g.KH, g.KW, g.SH, g.SW, g.PH, g.PW, in.stream());
              else
                  kernels::launch_conv2d_forward_kernel<float>(
                      static_cast<const float*>(in.data()), static_cast<const float*>(w.data()),
                      static_cast<const float*>(bptr), static_cast<float*>(out.data()), g.B,
                      g.IC, g.OC, g.IH, g.IW, g.KH, g.KW, g.SH, g.SW, g.PH, g.PW, in.stream());
              return out;
          },
          py::arg("input"), py::arg("weight"), py::arg("bias") = py::none(),
          py::arg("stride") = std::vector<int>{1, 1}, py::arg("padding") = std::vector<int>{0, 0});

    m.def("conv2d_backward_data",
          [](const Tensor& grad_output, const Tensor& weight, std::vector<int64_t> input_shape,
             std::vector<int> stride, std::vector<int> padding) {
              Tensor go = ensure_contiguous(grad_output), w = ensure_contiguous(weight);
              require_f32_or_f64(go, "conv2d_backward_data");
              if (w.dtype() != go.dtype())
                  throw std::runtime_error("conv2d_backward_data: grad_output and weight dtypes differ");
              ConvGeom g = conv_geom(input_shape, w.shape(), stride, padding);
              if (go.shape() != std::vector<int64_t>{g.B, g.OC, g.OH, g.OW})
                  throw std::runtime_error("conv2d_backward_data: grad_output shape mismatch");
              Tensor gi(input_shape, go.dtype());
              if (go.dtype() == DType::Float64)
                  kernels::launch_conv2d_backward_data_kernel<double>(
                      static_cast<const double*>(go.data()), static_cast<const double*>(w.data()),
                      static_cast<double*>(gi.data()), g.B, g.IC, g.OC, g.IH, g.IW, g.KH, g.KW,
                      g.SH, g.SW, g.PH, g.PW, go.stream());
              else
                  kernels::launch_conv2d_backward_data_kernel<float>(
                      static_cast<const float*>(go.data()), static_cast<const float*>(w.data()),
                      static_cast<float*>(gi.data()), g.B, g.IC, g.OC, g.IH, g.IW, g.KH, g.KW,
                      g.SH, g.SW, g.PH, g.PW, go.stream());
              return gi;
          },
          py::arg("grad_output"), py::arg("weight"), py::arg("input_shape"), py::arg("stride"),
          py::arg("padding"));

    m.def("conv2d_backward_weight",
          [](const Tensor& grad_output, const Tensor& input, std::vector<int64_t> weight_shape,
             std::vector<int> stride, std::vector<int> padding) {
              Tensor go = ensure_contiguous(grad_output), in = ensure_contiguous(input);
              require_f32_or_f64(go, "conv2d_backward_weight");
              if (in.dtype() != go.dtype())
                  throw std::runtime_error("conv2d_backward_weight: grad_output and input dtypes differ");
              ConvGeom g = conv_geom(in.shape(), weight_shape, stride, padding);
              if (go.shape() != std::vector<int64_t>{g.B, g.OC, g.OH, g.OW})
                  throw std::runtime_error("conv2d_backward_weight: grad_output shape mismatch");
              Tensor gw(weight_shape, go.dtype());
              if (go.dtype() == DType::Float64)
                  kernels::launch_conv2d_backward_weight_kernel<double>(
                      static_cast<const double*>(go.data()), static_cast<const double*>(in.data()),
                      static_cast<double*>(gw.data()), g.B, g.IC, g.OC, g.IH, g.IW, g.KH, g.KW,
                      g.SH, g.SW, g.PH, g.PW, go.stream());
              else
                  kernels::launch_conv2d_backward_weight_kernel<float>(
                      static_cast<const float*>(go.data()), static_cast<const float*>(in.data()),
                      static_cast<float*>(gw.data()), g.B, g.IC, g.OC, g.IH, g.IW, g.KH, g.KW,
                      g.SH, g.SW, g.PH, g.PW, go.stream());
              return gw;
          },
          py::arg("grad_output"), py::arg("input"), py::arg("weight_shape"), py::arg("stride"),
          py::arg("padding"));

    m.def("conv2d_backward_bias", [](const Tensor& grad_output) {
        Tensor go = ensure_contiguous(grad_output);
        require_f32_or_f64(go, "conv2d_backward_bias");
        if (go.ndim() != 4) throw std::runtime_error("conv2d_backward_bias: NCHW grad_output");
        const auto& s = go.shape();
        Tensor gb({s[1]}, go.dtype());
        if (go.dtype() == DType::Float64)
            kernels::launch_conv2d_backward_bias_kernel(static_cast<const double*>(go.data()),
                                                        static_cast<double*>(gb.data()), (int)s[0],
                                                        (int)s[1], (int)(s[2] * s[3]), go.stream());
        else
            kernels::launch_conv2d_backward_bias_kernel(static_cast<const float*>(go.data()),
                                                        static_cast<float*>(gb.data()), (int)s[0],
                                                        (int)s[1], (int)(s[2] * s[3]), go.stream());
        return gb;
    }, py::arg("grad_output"));

    m.def("device_info", []() {
        int device = 0;
        CUDEEP_CHECK_HIP(hipGetDevice(&device));
        hipDeviceProp_t p;
        CUDEEP_CHECK_HIP(hipGetDeviceProperties(&p, device));
        py::dict info;
        info["name"] = std::string(p.name);
        info["arch"] = std::string(p.gcnArchName);
        info["compute_capability"] = std::to_string(p.major) + "." + std::to_string(p.minor);
        info["total_memory_mb"] = (int64_t)(p.totalGlobalMem / (1024 * 1024));
        info["multiprocessors"] = p.multiProcessorCount;
        info["max_threads_per_block"] = p.maxThreadsPerBlock;
        info["warp_size"] = p.warpSize;
        info["clock_rate_mhz"] = p.clockRate / 1000;
        info["memory_clock_rate_mhz"] = p.memoryClockRate / 1000;
        info["memory_bus_width"] = p.memoryBusWidth;
        return info;
    });
}
