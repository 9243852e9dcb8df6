// Python module of the runtime: the surface of the reference's `vectorcore`
// module (python/bindings.cpp) with "hip" accepted as a device, plus hip
// diagnostics (pool statistics, per-launch profiler).
#include "vectorcore/vectorcore.hpp"
#include "vectorcore/detail/tensor_impl.hpp"

#include "vc_hip.h"

#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstring>
#include <optional>
#include <stdexcept>
#include <vector>

namespace py = pybind11;
using namespace vectorcore;

namespace {

Device parse_device(const std::string& name) {
    if (name == "cpu") return Device::cpu();
    if (name == "hip") return Device::hip();
    if (name == "metal" || name == "mps") return Device::metal();
    throw std::invalid_argument("device must be 'cpu', 'hip' or 'metal'");
}

Tensor from_python(const py::object& obj, bool requires_grad, const std::string& device_name) {
    const Device device = parse_device(device_name);
    if (py::isinstance<py::float_>(obj) || py::isinstance<py::int_>(obj))
        return Tensor::scalar(py::cast<float>(obj), requires_grad, device);
    auto arr = py::array_t<float, py::array::c_style | py::array::forcecast>::ensure(obj);
    if (!arr) throw std::invalid_argument("Tensor values must be a scalar or rectangular array-like object");
    Shape shape;
    for (py::ssize_t ax = 0; ax < arr.ndim(); ++ax) shape.push_back(static_cast<std::size_t>(arr.shape(ax)));
    std::vector<float> values(static_cast<std::size_t>(arr.size()));
    if (!values.empty()) std::memcpy(values.data(), arr.data(), values.size() * sizeof(float));
    return Tensor(std::move(values), std::move(shape), requires_grad, device);
}

py::array_t<float> to_numpy(const Tensor& t) {
    const auto values = t.to_vector();
    std::vector<py::ssize_t> shape(t.shape().begin(), t.shape().end());
    py::array_t<float> out(shape);
    if (!values.empty()) std::memcpy(out.mutable_data(), values.data(), values.size() * sizeof(float));
    return out;
}

// axis=None reduces everything; keepdim then keeps every axis with size 1.
template <class All, class Axis>
Tensor reduce(const Tensor& t, std::optional<std::int64_t> axis, bool keepdim, All all, Axis along) {
    if (axis) return along(t, *axis, keepdim);
    Tensor r = all(t);
    return keepdim ? r.reshape(Shape(t.ndim(), 1)) : r;
}

std::vector<std::size_t> targets_from(const py::object& obj) {
    if (py::isinstance<py::array>(obj)) {
        auto arr = py::array_t<std::int64_t, py::array::c_style | py::array::forcecast>::ensure(obj);
        std::vector<std::size_t> out(static_cast<std::size_t>(arr.size()));
        const std::int64_t* p = arr.data();
        for (std::size_t i = 0; i < out.size(); ++i) out[i] = static_cast<std::size_t>(p[i]);
        return out;
    }
    return py::cast<std::vector<std::size_t>>(obj);
}

void check(int status) {
    if (status != VC_HIP_OK) throw std::runtime_error(vc_hip_last_error());
}

}  // namespace

PYBIND11_MODULE(_vectorcore, m) {
    m.doc() = "VectorCore tensor and automatic differentiation runtime with an MI355X (HIP) device";

    py::class_<Tensor>(m, "Tensor")
        .def(py::init(&from_python), py::arg("values"), py::arg("requires_grad") = false, py::arg("device") = "cpu")
        .def_static("zeros", [](const Shape& s, bool rg, const std::string& d) { return Tensor::zeros(s, rg, parse_device(d)); },
                    py::arg("shape"), py::arg("requires_grad") = false, py::arg("device") = "cpu")
        .def_static("ones", [](const Shape& s, bool rg, const std::string& d) { return Tensor::ones(s, rg, parse_device(d)); },
                    py::arg("shape"), py::arg("requires_grad") = false, py::arg("device") = "cpu")
        .def_static("randn",
                    [](const Shape& s, bool rg, std::uint64_t seed, const std::string& d) {
                        return Tensor::randn(s, rg, seed, parse_device(d));
                    },
                    py::arg("shape"), py::arg("requires_grad") = false, py::arg("seed") = 0, py::arg("device") = "cpu")
        .def_property_readonly("shape", &Tensor::shape)
        .def_property_readonly("strides", &Tensor::strides)
        .def_property_readonly("ndim", &Tensor::ndim)
        .def_property_readonly("numel", &Tensor::numel)
        .def_property_readonly("device", [](const Tensor& t) { return t.device().str(); })
        .def_property_readonly("dtype", [](const Tensor&) { return "float32"; })
        .def_property("requires_grad", &Tensor::requires_grad, &Tensor::set_requires_grad)
        .def_property_readonly("is_leaf", &Tensor::is_leaf)
        .def_property_readonly("retains_grad", &Tensor::retains_grad)
        .def_property_readonly("_version", &Tensor::version)
        .def("retain_grad", &Tensor::retain_grad)
        .def_property_readonly("grad", [](const Tensor& t) -> py::object { return t.has_grad() ? py::cast(t.grad()) : py::none(); })
        .def("numpy", &to_numpy)
        .def("item", &Tensor::item)
        .def("at", &Tensor::at)
        .def("reshape", &Tensor::reshape)
        .def("flatten", &Tensor::flatten)
        .def("transpose", &Tensor::transpose)
        .def_property_readonly("T", &Tensor::transpose)
        .def("sum",
             [](const Tensor& t, std::optional<std::int64_t> axis, bool keepdim) {
                 return reduce(t, axis, keepdim, [](const Tensor& x) { return x.sum(); },
                               [](const Tensor& x, std::int64_t a, bool k) { return x.sum(a, k); });
             },
             py::arg("axis") = py::none(), py::arg("keepdim") = false)
        .def("mean",
             [](const Tensor& t, std::optional<std::int64_t> axis, bool keepdim) {
                 return reduce(t, axis, keepdim, [](const Tensor& x) { return x.mean(); },
                               [](const Tensor& x, std::int64_t a, bool k) { return x.mean(a, k); });
             },
             py::arg("axis") = py::none(), py::arg("keepdim") = false)
        .def("max",
             [](const Tensor& t, std::optional<std::int64_t> axis, bool keepdim) {
                 return reduce(t, axis, keepdim, [](const Tensor& x) { return x.max(); },
                               [](const Tensor& x, std::int64_t a, bool k) { return x.max(a, k); });
             },
             py::arg("axis") = py::none(), py::arg("keepdim") = false)
        .def("argmax",
             [](const Tensor& t, std::optional<std::int64_t> axis, bool keepdim) {
                 if (axis) return t.argmax(*axis, keepdim);
                 Tensor flat = t.flatten().argmax(0, false);
                 return keepdim ? flat.reshape(Shape(t.ndim(), 1)) : flat;
             },
             py::arg("axis") = py::none(), py::arg("keepdim") = false)
        .def("relu", &Tensor::relu)
        .def("sigmoid", &Tensor::sigmoid)
        .def("exp", py::overload_cast<>(&Tensor::exp, py::const_))
        .def("log", py::overload_cast<>(&Tensor::log, py::const_))
        .def("softmax", &Tensor::softmax, py::arg("axis") = -1)
        .def("log_softmax", &Tensor::log_softmax, py::arg("axis") = -1)
        .def("matmul", &Tensor::matmul)
        .def("to", [](const Tensor& t, const std::string& d) { return t.to(parse_device(d)); })
        .def("detach", &Tensor::detach)
        .def("backward", py::overload_cast<>(&Tensor::backward, py::const_))
        .def("backward", py::overload_cast<const Tensor&>(&Tensor::backward, py::const_))
        .def("zero_grad", &Tensor::zero_grad)
        .def("__repr__", &Tensor::repr)
        .def("__matmul__", &Tensor::matmul, py::is_operator())
        .def("__add__", [](const Tensor& a, const Tensor& b) { return a + b; }, py::is_operator())
        .def("__sub__", [](const Tensor& a, const Tensor& b) { return a - b; }, py::is_operator())
        .def("__mul__", [](const Tensor& a, const Tensor& b) { return a * b; }, py::is_operator())
        .def("__truediv__", [](const Tensor& a, const Tensor& b) { return a / b; }, py::is_operator())
        .def("__add__", [](const Tensor& a, float b) { return a + b; }, py::is_operator())
        .def("__sub__", [](const Tensor& a, float b) { return a - b; }, py::is_operator())
        .def("__mul__", [](const Tensor& a, float b) { return a * b; }, py::is_operator())
        .def("__truediv__", [](const Tensor& a, float b) { return a / b; }, py::is_operator())
        .def("__radd__", [](const Tensor& b, float a) { return a + b; }, py::is_operator())
        .def("__rsub__", [](const Tensor& b, float a) { return a - b; }, py::is_operator())
        .def("__rmul__", [](const Tensor& b, float a) { return a * b; }, py::is_operator())
        .def("__rtruediv__", [](const Tensor& b, float a) { return a / b; }, py::is_operator())
        .def("__neg__", [](const Tensor& v) { return -v; }, py::is_operator());

    py::class_<nn::Linear>(m, "Linear")
        .def(py::init<std::size_t, std::size_t, std::uint64_t>(), py::arg("in_features"), py::arg("out_features"),
             py::arg("seed") = 0)
        .def("__call__", &nn::Linear::operator())
        .def_readwrite("weight", &nn::Linear::weight)
        .def_readwrite("bias", &nn::Linear::bias);

    m.def("mse_loss", &nn::mse_loss);
    m.def("cross_entropy", [](const Tensor& logits, const py::object& targets) {
              return nn::cross_entropy(logits, targets_from(targets));
          },
          py::arg("logits"), py::arg("targets"),
          "Mean softmax cross-entropy of [batch, classes] logits and integer class targets.");
    m.def("softmax", [](const Tensor& t, std::int64_t axis) { return t.softmax(axis); }, py::arg("value"),
          py::arg("axis") = -1);
    m.def("log_softmax", [](const Tensor& t, std::int64_t axis) { return t.log_softmax(axis); }, py::arg("value"),
          py::arg("axis") = -1);
    m.def("sgd_step", [](std::vector<Tensor> params, float lr) {
        std::vector<Tensor*> ptrs;
        for (auto& p : params) ptrs.push_back(&p);
        nn::sgd_step(ptrs, lr);
    });
    m.def("zero_grad", [](std::vector<Tensor> params) {
        for (auto& p : params) p.zero_grad();
    });
    m.def("metal_available", &metal_available);
    m.def("metal_device_name", &metal_device_name);
    m.def("metal_gemm_kernel", [] { return std::string("unavailable"); });
    m.def("hip_available", &hip_available);
    m.def("hip_device_name", &hip_device_name);
    m.def("hip_gemm_kernel", [] { return HipBackend::instance().gemm_kernel(); },
          "Which HIP matmul kernel is active: 'mfma', 'simple' or 'unavailable'.");
    m.def(
        "hip_set_gemm_kernel",
        [](const std::string& name) {
            auto& b = HipBackend::instance();
            const std::string previous = b.gemm_kernel();
            b.set_gemm_kernel(name);
            return previous;
        },
        py::arg("name"),
        "Select the HIP matmul kernel for later products ('mfma' or 'simple', the portable FMA kernel); "
        "returns the previous one.");
    m.def("synchronize", &vectorcore::synchronize,
          "Wait for all queued device work; reading tensor values does this automatically.");

    m.def("hip_pool_stats", [] {
        vc_hip_pool_stats s{};
        check(vc_hip_pool_stats_get(&s));
        py::dict d;
        d["device_allocations"] = s.device_allocations;
        d["reuses"] = s.reuses;
        d["live_bytes"] = s.live_bytes;
        d["pooled_bytes"] = s.pooled_bytes;
        return d;
    });
    m.def(
        "hip_profile",
        [](bool enable, std::optional<std::vector<std::string>> labels) {
            std::string joined;
            if (labels)
                for (const auto& l : *labels) joined += (joined.empty() ? "" : ",") + l;
            check(vc_hip_profile_labels(labels ? joined.c_str() : nullptr));
            check(vc_hip_profile_enable(enable ? 1 : 0));
        },
        py::arg("enable"), py::arg("labels") = py::none());
    m.def(
        "_axpy_inplace",
        [](Tensor& target, std::size_t target_offset, const Tensor& source, std::size_t source_offset,
           std::size_t count, float alpha) {
            if (target.device() != Device::hip() || source.device() != Device::hip())
                throw std::invalid_argument("_axpy_inplace takes hip tensors");
            auto& storage = *target.impl()->storage;
            HipBackend::instance().axpy_inplace(storage, target.impl()->offset + target_offset, *source.impl()->storage,
                                                source.impl()->offset + source_offset, count, alpha);
            storage.bump_version();
        },
        py::arg("target"), py::arg("target_offset"), py::arg("source"), py::arg("source_offset"), py::arg("count"),
        py::arg("alpha"),
        "HipBackend::axpy_inplace on a range of two hip tensors' storages (the device interface's in-place "
        "update, for tests).");
    m.def(
        "hip_defer_products",
        [](std::optional<bool> enable) {
            auto& b = HipBackend::instance();
            const bool previous = b.defer_products();
            if (enable) b.set_defer_products(*enable);
            return previous;
        },
        py::arg("enable") = py::none(),
        "Whether 2-D hip products are computed on first use (fusing a following bias add and ReLU); "
        "sets it when `enable` is given and returns the previous setting.");
    m.def(
        "hip_strict_item",
        [](std::optional<bool> enable) {
            auto& b = HipBackend::instance();
            const bool previous = b.strict_item();
            if (enable) b.set_strict_item(*enable);
            return previous;
        },
        py::arg("enable") = py::none(),
        "Whether item()/to_vector() of a hip tensor first waits for all queued work and reports any asynchronous "
        "failure, as the reference's download does (otherwise a published loss waits for its producer only); "
        "sets it when `enable` is given and returns the previous setting.");
    m.def(
        "hip_fuse_elementwise",
        [](std::optional<bool> enable) {
            auto& b = HipBackend::instance();
            const bool previous = b.fuse_elementwise();
            if (enable) b.set_fuse_elementwise(*enable);
            return previous;
        },
        py::arg("enable") = py::none(),
        "Whether a hip backward pass evaluates its chains of elementwise gradient ops (and their bias column "
        "sums) as fused programs; sets it when `enable` is given and returns the previous setting.");
    m.def("hip_profile_reset", [] { check(vc_hip_profile_reset()); });
    m.def("hip_profile_read", [] {
        std::size_t n = 0;
        check(vc_hip_profile_count(&n));
        py::dict out;
        for (std::size_t i = 0; i < n; ++i) {
            const char* label = nullptr;
            std::uint64_t launches = 0;
            double ms = 0, flops = 0, bytes = 0;
            check(vc_hip_profile_entry(i, &label, &launches, &ms, &flops, &bytes));
            if (!launches) continue;
            py::dict e;
            e["launches"] = launches;
            e["ms"] = ms;
            e["flops"] = flops;
            e["bytes"] = bytes;
            out[label] = e;
        }
        return out;
    });
}
