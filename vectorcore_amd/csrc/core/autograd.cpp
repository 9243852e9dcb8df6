#include "vectorcore/autograd.hpp"

#include "vectorcore/cpu_backend.hpp"
#include "vectorcore/detail/tensor_impl.hpp"
#include "vectorcore/hip_backend.hpp"
#include "vectorcore/ops.hpp"

#include <stdexcept>
#include <string>

namespace vectorcore {

namespace {
thread_local bool t_grad_enabled = true;
}

NoGradGuard::NoGradGuard() : previous_(t_grad_enabled) { t_grad_enabled = false; }
NoGradGuard::~NoGradGuard() { t_grad_enabled = previous_; }
bool grad_enabled() { return t_grad_enabled; }

namespace detail {

namespace {
thread_local GradientOffer* t_gradient_offer = nullptr;
}

GradientOffer* gradient_offer() { return t_gradient_offer; }
void set_gradient_offer(GradientOffer* offer) { t_gradient_offer = offer; }

SavedTensor::SavedTensor(const Tensor& value) : tensor_(value.detach()), version_(value.version()) {}

Tensor SavedTensor::unpack() const {
    if (tensor_.version() != version_) {
        throw std::runtime_error(
            "a tensor needed for gradient computation was modified in place after it was used (saved version " +
            std::to_string(version_) + ", current version " + std::to_string(tensor_.version()) +
            "); run backward() before mutating it");
    }
    return tensor_;
}

std::optional<Tensor> SavedTensor::unpack_if_unchanged() const {
    if (tensor_.version() != version_) return std::nullopt;
    return tensor_;
}

void attach_grad_fn(Tensor& output, const std::vector<Tensor>& parents,
                    std::function<std::vector<Tensor>(const Tensor&)> backward) {
    if (!grad_enabled()) return;
    bool any = false;
    for (const auto& p : parents) any = any || p.requires_grad();
    if (!any) return;
    auto fn = std::make_shared<GradFn>();
    fn->parents.reserve(parents.size());
    for (const auto& p : parents) fn->parents.push_back(p.impl());
    fn->backward = std::move(backward);
    output.impl()->requires_grad = true;
    output.impl()->leaf = false;
    output.impl()->grad_fn = std::move(fn);
}

// Gradient of broadcasting (src/autograd.cpp:50-72): align the target to the
// gradient's rank with leading ones, sum (keepdim) every axis the forward
// stretched, in axis order, then reshape to the target.
Tensor sum_to_shape(const Tensor& gradient, const Shape& target_shape) {
    if (gradient.shape() == target_shape) return gradient;
    const Shape& src = gradient.shape();
    if (target_shape.size() > src.size())
        throw std::invalid_argument("cannot reduce " + shape_string(src) + " to larger rank " + shape_string(target_shape));
    const std::size_t lead = src.size() - target_shape.size();
    Tensor current = gradient;
    for (std::size_t ax = 0; ax < src.size(); ++ax) {
        const std::size_t want = ax < lead ? 1 : target_shape[ax - lead];
        if (want == src[ax]) continue;
        if (want != 1) throw std::invalid_argument("cannot reduce " + shape_string(src) + " to " + shape_string(target_shape));
        current = vectorcore::sum(current, static_cast<std::int64_t>(ax), true);
    }
    return current.reshape(target_shape);
}

// Expand a gradient back to a broadcast shape as value + 0 with an explicit
// output shape (src/autograd.cpp:74-91); like the reference this turns -0.0
// into +0.0.
Tensor broadcast_to(const Tensor& value, const Shape& target_shape) {
    if (value.shape() == target_shape) return value;
    (void)broadcast_shape(value.shape(), target_shape);  // validates
    const Tensor zero = Tensor::scalar(0.0F, false, value.device());
    std::shared_ptr<Storage> out;
    switch (value.device().type) {
        case DeviceType::CPU:
            out = make_cpu_storage(numel(target_shape));
            cpu::binary(value.data(), value.shape(), value.strides(), zero.data(), {}, {}, out->mutable_data(),
                        target_shape, cpu::BinaryOp::Add);
            break;
        case DeviceType::HIP:
            out = HipBackend::instance().binary(*value.impl()->storage, value.impl()->offset, value.shape(),
                                                value.strides(), *zero.impl()->storage, 0, {}, {}, target_shape,
                                                cpu::BinaryOp::Add);
            break;
        case DeviceType::METAL:
            throw std::runtime_error("Metal is unavailable: VectorCore was built without Apple Metal");
    }
    return make_tensor(std::move(out), target_shape, false);
}

}  // namespace detail

}  // namespace vectorcore
