// HipBackend and HipStorage over the C ABI (include/vc_hip.h).
//
// Ownership: a HipStorage owns one pooled device buffer and hands it back to
// the pool when the last tensor view dies; the library's single in-order
// stream makes that safe while queued kernels still use it. One-element
// storages created from host values (the scalar operands of
// src/tensor.cpp:323-330) keep their host value and touch the device only
// if a kernel needs them as a device operand.
#include "vectorcore/hip_backend.hpp"

#include "vc_hip.h"

#include <mutex>
#include <stdexcept>
#include <string>

namespace vectorcore {

namespace {

[[noreturn]] void throw_status(int status, const std::string& what) {
    const std::string message = what + ": " + vc_hip_last_error();
    switch (status) {
        case VC_HIP_ERR_INVALID_ARGUMENT: throw std::invalid_argument(message);
        case VC_HIP_ERR_OUT_OF_RANGE: throw std::out_of_range(message);
        case VC_HIP_ERR_OVERFLOW: throw std::overflow_error(message);
        default: throw std::runtime_error(message);
    }
}

inline void check(int status, const char* what) {
    if (status != VC_HIP_OK) throw_status(status, what);
}

class HipStorage final : public Storage {
public:
    // A fresh pooled buffer of `elements` floats (contents undefined).
    explicit HipStorage(std::size_t elements) : elements_(elements) {
        check(vc_hip_alloc(bytes(), &ptr_), "HIP allocation failed");
    }
    // A small tensor from host values: kept on the host until a kernel needs it.
    HipStorage(const float* values, std::size_t elements) : elements_(elements), shadow_(values, values + elements) {}

    ~HipStorage() override {
        if (ptr_) (void)vc_hip_release(ptr_);
    }
    HipStorage(const HipStorage&) = delete;
    HipStorage& operator=(const HipStorage&) = delete;

    [[nodiscard]] Device device() const noexcept override { return Device::hip(); }
    [[nodiscard]] std::size_t size() const noexcept override { return elements_; }

    float* ptr() const {
        std::lock_guard<std::mutex> lock(mu_);
        if (!ptr_) {
            check(vc_hip_alloc(bytes(), &ptr_), "HIP allocation failed");
            if (!shadow_.empty()) check(vc_hip_upload(ptr_, shadow_.data(), shadow_.size() * sizeof(float)), "HIP upload failed");
        }
        return static_cast<float*>(ptr_);
    }

    std::optional<float> host_scalar() const {
        std::lock_guard<std::mutex> lock(mu_);
        if (elements_ == 1 && shadow_valid_ && shadow_.size() == 1) return shadow_[0];
        return std::nullopt;
    }

    // Host copy readable without the device (no synchronisation needed).
    bool host_copy(std::size_t offset, float* dst, std::size_t n) const {
        std::lock_guard<std::mutex> lock(mu_);
        if (!shadow_valid_ || shadow_.empty()) return false;
        std::copy(shadow_.begin() + static_cast<std::ptrdiff_t>(offset),
                  shadow_.begin() + static_cast<std::ptrdiff_t>(offset + n), dst);
        return true;
    }

    void written_on_device() {
        (void)ptr();
        std::lock_guard<std::mutex> lock(mu_);
        shadow_valid_ = false;
    }

private:
    std::size_t bytes() const { return (elements_ ? elements_ : 1) * sizeof(float); }

    std::size_t elements_;
    mutable std::mutex mu_;
    mutable void* ptr_ = nullptr;
    std::vector<float> shadow_;
    bool shadow_valid_ = true;
};

constexpr std::size_t kHostKeptElements = 16;

const HipStorage& as_hip(const Storage& s) {
    const auto* h = dynamic_cast<const HipStorage*>(&s);
    if (!h) throw std::invalid_argument("expected HIP storage");
    return *h;
}

HipStorage& as_hip(Storage& s) {
    auto* h = dynamic_cast<HipStorage*>(&s);
    if (!h) throw std::invalid_argument("expected HIP storage");
    return *h;
}

float* dptr(const Storage& s, std::size_t offset) { return as_hip(s).ptr() + offset; }

std::shared_ptr<HipStorage> fresh(std::size_t elements) { return std::make_shared<HipStorage>(elements); }

void require(const HipBackend& b) {
    if (!b.available()) throw std::runtime_error("HIP backend unavailable: " + b.last_error());
}

int binary_code(cpu::BinaryOp op) { return static_cast<int>(op); }

}  // namespace

HipBackend& HipBackend::instance() {
    static HipBackend backend;
    return backend;
}

bool HipBackend::available() const noexcept { return vc_hip_available() != 0; }
std::string HipBackend::device_name() const { return vc_hip_device_name(); }
std::string HipBackend::last_error() const { return vc_hip_last_error(); }
std::string HipBackend::gemm_kernel() const { return vc_hip_gemm_kernel(); }

std::shared_ptr<Storage> HipBackend::allocate(std::size_t elements) {
    require(*this);
    return fresh(elements);
}

std::shared_ptr<Storage> HipBackend::upload(const float* data, std::size_t elements) {
    require(*this);
    if (elements <= kHostKeptElements && elements > 0) return std::make_shared<HipStorage>(data, elements);
    auto out = fresh(elements);
    if (elements) check(vc_hip_upload(out->ptr(), data, elements * sizeof(float)), "HIP upload failed");
    return out;
}

void HipBackend::download(const Storage& source, std::size_t offset, float* destination, std::size_t elements) {
    if (offset + elements > source.size()) throw std::out_of_range("HIP download exceeds storage");
    const auto& h = as_hip(source);
    if (h.host_copy(offset, destination, elements)) return;
    check(vc_hip_download(destination, h.ptr() + offset, elements * sizeof(float)), "HIP command failed");
}

std::shared_ptr<Storage> HipBackend::binary(const Storage& a, std::size_t a_offset, const Shape& a_shape,
                                            const Strides& a_strides, const Storage& b, std::size_t b_offset,
                                            const Shape& b_shape, const Strides& b_strides, const Shape& out_shape,
                                            cpu::BinaryOp operation) {
    require(*this);
    if (out_shape.size() > 8 || a_shape.size() > 8 || b_shape.size() > 8)
        throw std::invalid_argument("HIP broadcasting supports at most 8 dimensions");
    const std::size_t count = numel(out_shape);
    // Both operands host-known scalars: the same fp32 operation on the host.
    if (count == 1 && numel(a_shape) == 1 && numel(b_shape) == 1) {
        const auto sa = hip_host_scalar(a), sb = hip_host_scalar(b);
        if (sa && sb) {
            float r = 0.0F;
            switch (operation) {
                case cpu::BinaryOp::Add: r = *sa + *sb; break;
                case cpu::BinaryOp::Subtract: r = *sa - *sb; break;
                case cpu::BinaryOp::Multiply: r = *sa * *sb; break;
                case cpu::BinaryOp::Divide: r = *sa / *sb; break;
            }
            return std::make_shared<HipStorage>(&r, 1);
        }
    }
    // A host-known scalar against an output-shaped operand: the value goes in
    // the kernel arguments.
    if (a_shape == out_shape && numel(b_shape) == 1) {
        if (auto s = hip_host_scalar(b)) return binary_scalar(a, a_offset, count, *s, false, operation);
    }
    if (b_shape == out_shape && numel(a_shape) == 1) {
        if (auto s = hip_host_scalar(a)) return binary_scalar(b, b_offset, count, *s, true, operation);
    }
    auto out = fresh(count);
    if (count == 0) return out;
    check(vc_hip_binary(dptr(a, a_offset), a_shape.data(), a_strides.data(), a_shape.size(), dptr(b, b_offset),
                        b_shape.data(), b_strides.data(), b_shape.size(), out->ptr(), out_shape.data(),
                        out_shape.size(), binary_code(operation)),
          "HIP binary op failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::binary_scalar(const Storage& a, std::size_t a_offset, std::size_t count, float s,
                                                   bool scalar_first, cpu::BinaryOp operation) {
    require(*this);
    auto out = fresh(count);
    if (count == 0) return out;
    check(vc_hip_binary_scalar(dptr(a, a_offset), count, s, scalar_first ? 1 : 0, out->ptr(), binary_code(operation)),
          "HIP binary op failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::unary(const Storage& input, std::size_t offset, std::size_t count,
                                           cpu::UnaryOp operation) {
    require(*this);
    auto out = fresh(count);
    if (count == 0) return out;
    check(vc_hip_unary(dptr(input, offset), out->ptr(), count, static_cast<int>(operation)), "HIP unary op failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::matmul(const Storage& a, std::size_t a_offset, const Storage& b,
                                            std::size_t b_offset, std::size_t m, std::size_t k, std::size_t n,
                                            const std::vector<std::size_t>& a_offsets,
                                            const std::vector<std::size_t>& b_offsets, bool trans_a, bool trans_b) {
    require(*this);
    if (a_offsets.size() != b_offsets.size() || a_offsets.empty())
        throw std::invalid_argument("HIP matmul needs one A and B offset per batch");
    const std::size_t batch = a_offsets.size();
    auto out = fresh(batch * m * n);
    if (batch * m * n == 0) return out;
    if (k == 0) {  // empty inner dimension: the product is zero
        check(vc_hip_fill(out->ptr(), batch * m * n, 0.0F), "HIP fill failed");
        return out;
    }
    check(vc_hip_matmul(dptr(a, a_offset), dptr(b, b_offset), out->ptr(), m, k, n, a_offsets.data(),
                        b_offsets.data(), batch, trans_a ? 1 : 0, trans_b ? 1 : 0),
          "HIP matmul failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::matmul_relu_mask(const Storage& a, std::size_t a_offset, const Storage& b,
                                                      std::size_t b_offset, std::size_t m, std::size_t k, std::size_t n,
                                                      const std::vector<std::size_t>& a_offsets,
                                                      const std::vector<std::size_t>& b_offsets, bool trans_a,
                                                      bool trans_b, const Storage& relu_input,
                                                      std::size_t relu_offset) {
    require(*this);
    if (a_offsets.size() != b_offsets.size() || a_offsets.empty())
        throw std::invalid_argument("HIP matmul needs one A and B offset per batch");
    const std::size_t batch = a_offsets.size();
    auto out = fresh(batch * m * n);
    if (batch * m * n == 0) return out;
    if (k == 0) {  // empty inner dimension: the product, masked or not, is +0
        check(vc_hip_fill(out->ptr(), batch * m * n, 0.0F), "HIP fill failed");
        return out;
    }
    check(vc_hip_matmul_relu_mask(dptr(a, a_offset), dptr(b, b_offset), out->ptr(), m, k, n, a_offsets.data(),
                                  b_offsets.data(), batch, trans_a ? 1 : 0, trans_b ? 1 : 0,
                                  dptr(relu_input, relu_offset)),
          "HIP matmul failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::matmul_reduce(const Storage& a, std::size_t a_offset, const Storage& b,
                                                   std::size_t b_offset, std::size_t m, std::size_t k, std::size_t n,
                                                   std::size_t count, std::size_t a_stride, std::size_t b_stride,
                                                   bool trans_a, bool trans_b) {
    require(*this);
    auto out = fresh(m * n);
    if (m * n == 0) return out;
    if (k == 0 || count == 0) {
        check(vc_hip_fill(out->ptr(), m * n, 0.0F), "HIP fill failed");
        return out;
    }
    check(vc_hip_matmul_reduce(dptr(a, a_offset), dptr(b, b_offset), out->ptr(), m, k, n, count, a_stride, b_stride,
                               trans_a ? 1 : 0, trans_b ? 1 : 0),
          "HIP matmul failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::transpose_last2(const Storage& input, std::size_t offset, std::size_t batch,
                                                     std::size_t rows, std::size_t cols) {
    require(*this);
    auto out = fresh(batch * rows * cols);
    if (batch * rows * cols == 0) return out;
    check(vc_hip_transpose_last2(dptr(input, offset), out->ptr(), batch, rows, cols), "HIP transpose failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::reduce_sum(const Storage& input, std::size_t offset, std::size_t count) {
    require(*this);
    auto out = fresh(1);
    check(vc_hip_reduce_sum(count ? dptr(input, offset) : nullptr, count, out->ptr()), "HIP sum failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::reduce_axis(const Storage& input, std::size_t offset, std::size_t outer,
                                                 std::size_t length, std::size_t inner, cpu::ReduceOp operation) {
    require(*this);
    if (length == 0 && operation != cpu::ReduceOp::Sum)
        throw std::invalid_argument("max/argmax over an empty axis is undefined");
    auto out = fresh(outer * inner);
    if (outer * inner == 0) return out;
    check(vc_hip_reduce_axis(outer * length * inner != 0 ? dptr(input, offset) : nullptr, out->ptr(), outer, length, inner,
                             static_cast<int>(operation)),
          "HIP axis reduction failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::scatter_axis(const Storage& values, std::size_t values_offset,
                                                  const Storage& indices, std::size_t indices_offset,
                                                  std::size_t outer, std::size_t length, std::size_t inner) {
    require(*this);
    auto out = fresh(outer * length * inner);
    if (outer * length * inner == 0) return out;
    check(vc_hip_scatter_axis(dptr(values, values_offset), dptr(indices, indices_offset), out->ptr(), outer, length,
                              inner),
          "HIP scatter failed");
    return out;
}

void HipBackend::axpy_inplace(Storage& target, std::size_t target_offset, const Storage& source,
                              std::size_t source_offset, std::size_t count, float alpha) {
    require(*this);
    if (target_offset + count > target.size() || source_offset + count > source.size())
        throw std::out_of_range("HIP axpy exceeds storage");
    auto& t = as_hip(target);
    t.written_on_device();
    if (count == 0) return;
    check(vc_hip_axpy(t.ptr() + target_offset, dptr(source, source_offset), count, alpha), "HIP axpy failed");
}

void HipBackend::axpy_batch(const std::vector<AxpyItem>& items, float alpha) {
    require(*this);
    std::vector<float*> targets;
    std::vector<const float*> sources;
    std::vector<std::size_t> counts;
    for (const AxpyItem& it : items) {
        if (it.target_offset + it.count > it.target->size() || it.source_offset + it.count > it.source->size())
            throw std::out_of_range("HIP axpy exceeds storage");
        auto& t = as_hip(*it.target);
        t.written_on_device();
        if (it.count == 0) continue;
        targets.push_back(t.ptr() + it.target_offset);
        sources.push_back(dptr(*it.source, it.source_offset));
        counts.push_back(it.count);
    }
    if (targets.empty()) return;
    check(vc_hip_axpy_batch(targets.data(), sources.data(), counts.data(), targets.size(), alpha), "HIP axpy failed");
}

void HipBackend::synchronize() {
    if (!available()) return;
    check(vc_hip_synchronize(), "HIP command failed");
}

std::shared_ptr<Storage> HipBackend::fill(std::size_t count, float value) {
    require(*this);
    auto out = fresh(count);
    if (count) check(vc_hip_fill(out->ptr(), count, value), "HIP fill failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::activation_backward(Activation kind, const Storage& grad, std::size_t grad_offset,
                                                         const Storage& saved, std::size_t saved_offset,
                                                         std::size_t count) {
    require(*this);
    auto out = fresh(count);
    if (count == 0) return out;
    const float* g = dptr(grad, grad_offset);
    const float* s = dptr(saved, saved_offset);
    int status = VC_HIP_OK;
    switch (kind) {
        case Activation::Relu: status = vc_hip_relu_backward(g, s, out->ptr(), count); break;
        case Activation::Sigmoid: status = vc_hip_sigmoid_backward(g, s, out->ptr(), count); break;
        case Activation::Exp: status = vc_hip_exp_backward(g, s, out->ptr(), count); break;
        case Activation::Log: status = vc_hip_log_backward(g, s, out->ptr(), count); break;
    }
    check(status, "HIP activation backward failed");
    return out;
}

std::pair<std::shared_ptr<Storage>, std::shared_ptr<Storage>> HipBackend::divide_backward(
    const Storage& grad, std::size_t grad_offset, const Storage& a, std::size_t a_offset, const Shape& a_shape,
    const Strides& a_strides, const Storage& b, std::size_t b_offset, const Shape& b_shape, const Strides& b_strides,
    const Shape& out_shape, bool need_a, bool need_b) {
    require(*this);
    const std::size_t count = numel(out_shape);
    std::shared_ptr<HipStorage> ga = need_a ? fresh(count) : nullptr;
    std::shared_ptr<HipStorage> gb = need_b ? fresh(count) : nullptr;
    if (count && (need_a || need_b)) {
        check(vc_hip_div_backward(dptr(grad, grad_offset), dptr(a, a_offset), a_shape.data(), a_strides.data(),
                                  a_shape.size(), dptr(b, b_offset), b_shape.data(), b_strides.data(), b_shape.size(),
                                  out_shape.data(), out_shape.size(), ga ? ga->ptr() : nullptr,
                                  gb ? gb->ptr() : nullptr),
              "HIP divide backward failed");
    }
    return {ga, gb};
}

namespace {
// The last class-index vector uploaded. Device copies of targets are never
// written, so a loss over the same targets as the previous one (a fixed
// batch) reuses that buffer instead of copying it again. Never destroyed: it
// must not release device memory after the HIP runtime has shut down.
struct TargetsCache {
    std::mutex mu;
    std::vector<std::int32_t> host;
    std::shared_ptr<Storage> device;
};
TargetsCache& targets_cache() {
    static auto* cache = new TargetsCache();
    return *cache;
}
}  // namespace

std::shared_ptr<Storage> HipBackend::upload_targets(const std::vector<std::size_t>& targets) {
    require(*this);
    std::vector<std::int32_t> t(targets.size());
    for (std::size_t i = 0; i < targets.size(); ++i) t[i] = static_cast<std::int32_t>(targets[i]);
    TargetsCache& cache = targets_cache();
    std::lock_guard<std::mutex> lock(cache.mu);
    if (cache.device && cache.host == t) return cache.device;
    auto out = fresh(targets.size());  // int32 and float have the same width
    if (!t.empty()) check(vc_hip_upload(out->ptr(), t.data(), t.size() * sizeof(std::int32_t)), "HIP upload failed");
    cache.host = std::move(t);
    cache.device = out;
    return out;
}

std::pair<std::shared_ptr<Storage>, std::shared_ptr<Storage>> HipBackend::cross_entropy_forward(
    const Storage& logits, std::size_t logits_offset, const Storage& targets, std::size_t rows, std::size_t classes) {
    require(*this);
    auto loss = fresh(1);
    auto stats = fresh(2 * rows);
    check(vc_hip_xent_forward(dptr(logits, logits_offset), reinterpret_cast<const std::int32_t*>(as_hip(targets).ptr()),
                              rows, classes, stats->ptr(), loss->ptr()),
          "HIP cross-entropy failed");
    return {loss, stats};
}

std::shared_ptr<Storage> HipBackend::cross_entropy_backward(const Storage& logits, std::size_t logits_offset,
                                                            const Storage& targets, const Storage& row_stats,
                                                            const Storage& grad_loss, std::size_t grad_offset,
                                                            std::size_t rows, std::size_t classes) {
    require(*this);
    auto out = fresh(rows * classes);
    check(vc_hip_xent_backward(dptr(logits, logits_offset),
                               reinterpret_cast<const std::int32_t*>(as_hip(targets).ptr()), as_hip(row_stats).ptr(),
                               dptr(grad_loss, grad_offset), rows, classes, out->ptr()),
          "HIP cross-entropy backward failed");
    return out;
}

std::optional<float> hip_host_scalar(const Storage& storage) {
    const auto* h = dynamic_cast<const HipStorage*>(&storage);
    return h ? h->host_scalar() : std::nullopt;
}

bool hip_available() { return HipBackend::instance().available(); }
std::string hip_device_name() { return HipBackend::instance().device_name(); }

}  // namespace vectorcore
