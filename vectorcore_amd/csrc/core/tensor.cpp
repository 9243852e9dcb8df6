#include "vectorcore/tensor.hpp"

#include "vectorcore/autograd.hpp"
#include "vectorcore/detail/tensor_impl.hpp"
#include "vectorcore/hip_backend.hpp"
#include "vectorcore/metal_backend.hpp"
#include "vectorcore/ops.hpp"
#include "vectorcore/storage.hpp"

#include <algorithm>
#include <iomanip>
#include <optional>
#include <random>
#include <sstream>
#include <stdexcept>
#include <unordered_map>
#include <unordered_set>
#include <utility>

namespace vectorcore {

std::string Device::str() const {
    switch (type) {
        case DeviceType::CPU: return "cpu";
        case DeviceType::METAL: return "metal";
        case DeviceType::HIP: return "hip";
    }
    return "unknown";
}

bool metal_available() { return false; }
std::string metal_device_name() { return "unavailable"; }
void synchronize() { HipBackend::instance().synchronize(); }

namespace {

[[noreturn]] void metal_unavailable() {
    throw std::runtime_error("Metal is unavailable: VectorCore was built without Apple Metal");
}

void require_hip() {
    auto& hip = HipBackend::instance();
    if (!hip.available()) throw std::runtime_error("HIP is unavailable: " + hip.last_error());
}

std::shared_ptr<Storage> storage_from_host(const float* values, std::size_t count, Device device) {
    switch (device.type) {
        case DeviceType::CPU: return make_cpu_storage(values, count);
        case DeviceType::HIP: require_hip(); return HipBackend::instance().upload(values, count);
        case DeviceType::METAL: metal_unavailable();
    }
    throw std::logic_error("unknown device");
}

}  // namespace

namespace detail {

Tensor from_impl(std::shared_ptr<TensorImpl> impl) { return Tensor(std::move(impl)); }

Tensor make_tensor(std::shared_ptr<Storage> storage, Shape shape, bool requires_grad) {
    if (!storage) throw std::invalid_argument("tensor storage cannot be null");
    if (storage->size() < numel(shape)) throw std::invalid_argument("storage is smaller than tensor shape");
    auto impl = std::make_shared<TensorImpl>();
    impl->storage = std::move(storage);
    impl->strides = contiguous_strides(shape);
    impl->shape = std::move(shape);
    impl->requires_grad = requires_grad;
    return from_impl(std::move(impl));
}

}  // namespace detail

Tensor::Tensor() : Tensor(std::vector<float>{0.0F}, Shape{}) {}

Tensor::Tensor(std::shared_ptr<detail::TensorImpl> impl) : impl_(std::move(impl)) {
    if (!impl_) throw std::invalid_argument("TensorImpl cannot be null");
}

Tensor::Tensor(std::vector<float> values, Shape shape, bool requires_grad, Device device) {
    const std::size_t count = vectorcore::numel(shape);
    if (values.size() != count)
        throw std::invalid_argument("received " + std::to_string(values.size()) + " values for shape " +
                                    shape_string(shape) + " containing " + std::to_string(count) + " elements");
    impl_ = detail::make_tensor(storage_from_host(values.data(), count, device), std::move(shape), requires_grad).impl();
}

Tensor Tensor::scalar(float value, bool requires_grad, Device device) { return Tensor({value}, {}, requires_grad, device); }

namespace {
Tensor filled(const Shape& shape, float value, bool requires_grad, Device device) {
    const std::size_t n = numel(shape);
    if (device == Device::hip() && n > 16) {  // large: fill on the device, no host copy
        require_hip();
        return detail::make_tensor(HipBackend::instance().fill(n, value), shape, requires_grad);
    }
    return Tensor(std::vector<float>(n, value), shape, requires_grad, device);
}
}  // namespace

Tensor Tensor::zeros(const Shape& shape, bool requires_grad, Device device) {
    return filled(shape, 0.0F, requires_grad, device);
}

Tensor Tensor::ones(const Shape& shape, bool requires_grad, Device device) {
    return filled(shape, 1.0F, requires_grad, device);
}

Tensor Tensor::randn(const Shape& shape, bool requires_grad, std::uint64_t seed, Device device) {
    std::mt19937_64 gen(seed);
    std::normal_distribution<float> normal(0.0F, 1.0F);
    std::vector<float> v(vectorcore::numel(shape));
    for (float& x : v) x = normal(gen);
    return Tensor(std::move(v), shape, requires_grad, device);
}

const Shape& Tensor::shape() const { return impl_->shape; }
const Strides& Tensor::strides() const { return impl_->strides; }
std::size_t Tensor::ndim() const { return impl_->shape.size(); }
std::size_t Tensor::numel() const { return vectorcore::numel(impl_->shape); }
Device Tensor::device() const { return impl_->storage->device(); }
DType Tensor::dtype() const { return impl_->dtype; }
bool Tensor::is_contiguous() const { return vectorcore::is_contiguous(shape(), strides()); }
bool Tensor::requires_grad() const { return impl_->requires_grad; }
bool Tensor::is_leaf() const { return impl_->leaf; }
bool Tensor::retains_grad() const { return impl_->retains_grad; }
std::uint64_t Tensor::version() const { return impl_->storage->version(); }

void Tensor::retain_grad() {
    if (!impl_->requires_grad) throw std::runtime_error("retain_grad() requires a tensor that requires gradients");
    if (!impl_->leaf) impl_->retains_grad = true;
}

void Tensor::set_requires_grad(bool value) {
    if (!impl_->leaf) throw std::runtime_error("requires_grad can only be changed on leaf tensors");
    impl_->requires_grad = value;
    if (!value) impl_->grad.reset();
}

const float* Tensor::data() const {
    if (device() != Device::cpu()) throw std::runtime_error("data() is only valid for CPU tensors; use to(CPU)");
    return impl_->storage->data() + impl_->offset;
}

float* Tensor::mutable_data() {
    if (device() != Device::cpu()) throw std::runtime_error("mutable_data() is only valid for CPU tensors; use to(CPU)");
    impl_->storage->bump_version();  // a writable pointer counts as an in-place write
    return impl_->storage->mutable_data() + impl_->offset;
}

std::vector<float> Tensor::to_vector() const {
    std::vector<float> out(numel());
    switch (device().type) {
        case DeviceType::CPU: std::copy(data(), data() + out.size(), out.begin()); break;
        case DeviceType::HIP:
            HipBackend::instance().download(*impl_->storage, impl_->offset, out.data(), out.size());
            break;
        case DeviceType::METAL: metal_unavailable();
    }
    return out;
}

float Tensor::item() const {
    if (numel() != 1) throw std::runtime_error("item() requires a one-element tensor");
    return to_vector().front();
}

namespace {
std::size_t flat_index(const Tensor& t, const std::vector<std::size_t>& idx) {
    if (idx.size() != t.ndim()) throw std::out_of_range("index rank does not match tensor rank");
    std::size_t off = 0;
    for (std::size_t ax = 0; ax < idx.size(); ++ax) {
        if (idx[ax] >= t.shape()[ax]) throw std::out_of_range("tensor index out of bounds");
        off += idx[ax] * t.strides()[ax];
    }
    return off;
}
}  // namespace

float Tensor::at(const std::vector<std::size_t>& indices) const {
    const std::size_t off = flat_index(*this, indices);
    if (device() == Device::cpu()) return data()[off];
    return to_vector()[off];
}

void Tensor::set_at(const std::vector<std::size_t>& indices, float value) {
    if (device() != Device::cpu()) throw std::runtime_error("set_at is only supported on CPU tensors");
    const std::size_t off = flat_index(*this, indices);
    mutable_data()[off] = value;
}

Tensor Tensor::to(Device target) const {
    if (target == device()) return *this;
    if (target == Device::metal() || device() == Device::metal()) metal_unavailable();
    const auto values = to_vector();
    auto output = detail::make_tensor(storage_from_host(values.data(), values.size(), target), shape(), false);
    const Device source = device();
    detail::attach_grad_fn(output, {*this}, [source](const Tensor& g) { return std::vector<Tensor>{g.to(source)}; });
    return output;
}

Tensor Tensor::reshape(const Shape& new_shape) const {
    if (vectorcore::numel(new_shape) != numel())
        throw std::invalid_argument("cannot reshape " + shape_string(shape()) + " to " + shape_string(new_shape));
    if (!is_contiguous()) throw std::runtime_error("reshape requires contiguous storage");
    auto view = std::make_shared<detail::TensorImpl>();
    view->storage = impl_->storage;
    view->shape = new_shape;
    view->strides = contiguous_strides(new_shape);
    view->offset = impl_->offset;
    auto output = detail::from_impl(std::move(view));
    const Shape original = shape();
    detail::attach_grad_fn(output, {*this}, [original](const Tensor& g) { return std::vector<Tensor>{g.reshape(original)}; });
    return output;
}

Tensor Tensor::flatten() const { return reshape({numel()}); }
Tensor Tensor::transpose() const { return vectorcore::transpose(*this); }
Tensor Tensor::sum() const { return vectorcore::sum(*this); }
Tensor Tensor::mean() const { return vectorcore::mean(*this); }
Tensor Tensor::relu() const { return vectorcore::relu(*this); }
Tensor Tensor::sigmoid() const { return vectorcore::sigmoid(*this); }
Tensor Tensor::exp() const { return vectorcore::exp(*this); }
Tensor Tensor::log() const { return vectorcore::log(*this); }
Tensor Tensor::sum(std::int64_t axis, bool keepdim) const { return vectorcore::sum(*this, axis, keepdim); }
Tensor Tensor::mean(std::int64_t axis, bool keepdim) const { return vectorcore::mean(*this, axis, keepdim); }
Tensor Tensor::max() const { return vectorcore::max(*this); }
Tensor Tensor::max(std::int64_t axis, bool keepdim) const { return vectorcore::max(*this, axis, keepdim); }
Tensor Tensor::argmax(std::int64_t axis, bool keepdim) const { return vectorcore::argmax(*this, axis, keepdim); }
Tensor Tensor::softmax(std::int64_t axis) const { return vectorcore::softmax(*this, axis); }
Tensor Tensor::log_softmax(std::int64_t axis) const { return vectorcore::log_softmax(*this, axis); }
Tensor Tensor::matmul(const Tensor& other) const { return vectorcore::matmul(*this, other); }

Tensor Tensor::detach() const {
    auto d = std::make_shared<detail::TensorImpl>();
    d->storage = impl_->storage;
    d->shape = impl_->shape;
    d->strides = impl_->strides;
    d->offset = impl_->offset;
    d->dtype = impl_->dtype;
    return detail::from_impl(std::move(d));
}

bool Tensor::has_grad() const { return static_cast<bool>(impl_->grad); }

Tensor Tensor::grad() const {
    if (!impl_->grad) throw std::runtime_error("tensor has no gradient");
    return detail::from_impl(impl_->grad);
}

void Tensor::zero_grad() { impl_->grad.reset(); }

void Tensor::backward() const {
    if (numel() != 1) throw std::runtime_error("backward() without a gradient requires a scalar tensor");
    backward(Tensor::ones(shape(), false, device()));
}

namespace {
void run_backward(const std::shared_ptr<detail::TensorImpl>& root,
                  const std::vector<std::shared_ptr<detail::TensorImpl>>& order, const Tensor& gradient);
}  // namespace

// Reverse-mode engine (the semantics of src/tensor.cpp:251-301): nodes in
// depth-first post-order over grad_fn parents, walked in reverse; each node's
// summed upstream gradient is consumed and dropped once used; leaves and
// retain_grad nodes store it in .grad; contributions to one node are added
// with operator+ in arrival order.
void Tensor::backward(const Tensor& gradient) const {
    if (!requires_grad()) throw std::runtime_error("cannot call backward on a tensor without gradients");
    if (gradient.shape() != shape()) throw std::invalid_argument("backward gradient shape mismatch");
    if (gradient.device() != device()) throw std::invalid_argument("backward gradient device mismatch");

    // Iterative DFS with the same post-order a recursive visit would give.
    std::vector<std::shared_ptr<detail::TensorImpl>> order;
    std::unordered_set<detail::TensorImpl*> seen;
    std::vector<std::pair<std::shared_ptr<detail::TensorImpl>, std::size_t>> stack;
    seen.insert(impl_.get());
    stack.emplace_back(impl_, 0);
    while (!stack.empty()) {
        auto& [node, next] = stack.back();
        const auto* parents = node->grad_fn ? &node->grad_fn->parents : nullptr;
        if (parents && next < parents->size()) {
            auto parent = (*parents)[next++];
            if (seen.insert(parent.get()).second) stack.emplace_back(std::move(parent), 0);
            continue;
        }
        order.push_back(node);
        stack.pop_back();
    }

    NoGradGuard guard;
    // On hip, the elementwise rules of this pass record expressions; the ones
    // still referenced when the pass ends (leaf and retained gradients) are
    // computed together by flush_elementwise below.
    std::optional<HipBackend::ElementwiseScope> fusion;
    if (gradient.device() == Device::hip()) fusion.emplace();
    run_backward(impl_, order, gradient);
    if (fusion) HipBackend::instance().flush_elementwise();
}

namespace {

// The node loop of Tensor::backward over `order` (depth-first post-order from
// root), seeded with `gradient` at root.
void run_backward(const std::shared_ptr<detail::TensorImpl>& root,
                  const std::vector<std::shared_ptr<detail::TensorImpl>>& order, const Tensor& gradient) {
    // How many graph nodes feed a gradient to each node.
    std::unordered_map<detail::TensorImpl*, int> consumers;
    for (const auto& node : order)
        if (node->grad_fn)
            for (const auto& parent : node->grad_fn->parents) ++consumers[parent.get()];

    std::unordered_map<detail::TensorImpl*, Tensor> pending;
    std::unordered_set<detail::TensorImpl*> premasked;  // ReLU outputs whose gradient arrived masked
    pending.emplace(root.get(), gradient.detach());
    for (auto it = order.rbegin(); it != order.rend(); ++it) {
        const auto& node = *it;
        auto found = pending.find(node.get());
        if (found == pending.end()) continue;
        const Tensor upstream = found->second;
        pending.erase(found);
        if (node->requires_grad && (node->leaf || node->retains_grad)) {
            node->grad = node->grad ? (detail::from_impl(node->grad) + upstream).detach().impl() : upstream.detach().impl();
        }
        if (!node->grad_fn) continue;
        std::vector<Tensor> grads;
        if (premasked.count(node.get())) {
            grads.push_back(upstream);  // the producer already applied this ReLU's rule
        } else {
            // Offer the ReLU mask of parent 0 when its gradient comes from this
            // node alone and is not kept: the rule may fuse it into its kernel
            // (hip products do). The gradient is the same either way.
            const auto& first = node->grad_fn->parents.empty() ? nullptr : node->grad_fn->parents[0];
            detail::GradientOffer offer;
            const bool on_hip = upstream.device() == Device::hip();
            const bool offered = first && on_hip && first->grad_fn && first->grad_fn->relu_mask &&
                                 first->requires_grad && !first->leaf && !first->retains_grad &&
                                 consumers[first.get()] == 1;
            if (offered) offer.relu_mask = first->grad_fn->relu_mask;
            // Will parent 0's gradient reach a row-bias add unchanged (that add
            // is parent 0, or the input of the ReLU whose mask is offered), the
            // add consumed by nothing else and its bias needing a gradient?
            const auto& add = offered ? (first->grad_fn->parents.empty() ? nullptr : first->grad_fn->parents[0]) : first;
            const int bias = on_hip && add && add->grad_fn ? add->grad_fn->row_bias_operand : -1;
            offer.column_sum_wanted = bias >= 0 && !add->leaf && !add->retains_grad && consumers[add.get()] == 1 &&
                                      add->grad_fn->parents[static_cast<std::size_t>(bias)]->requires_grad;
            if (offered || offer.column_sum_wanted) detail::set_gradient_offer(&offer);
            try {
                grads = node->grad_fn->backward(upstream);
            } catch (...) {
                detail::set_gradient_offer(nullptr);
                throw;
            }
            detail::set_gradient_offer(nullptr);
            if (offered && offer.taken) premasked.insert(first.get());
        }
        if (grads.size() != node->grad_fn->parents.size())
            throw std::logic_error("autograd function returned the wrong number of gradients");
        for (std::size_t i = 0; i < grads.size(); ++i) {
            const auto& parent = node->grad_fn->parents[i];
            if (!parent->requires_grad) continue;
            auto existing = pending.find(parent.get());
            if (existing == pending.end()) pending.emplace(parent.get(), grads[i].detach());
            else existing->second = existing->second + grads[i];
        }
    }
}

}  // namespace

std::string Tensor::repr() const {
    std::ostringstream s;
    s << "Tensor(shape=" << shape_string(shape()) << ", dtype='float32', device='" << device().str()
      << "', requires_grad=" << (requires_grad() ? "true" : "false") << ", values=[";
    const auto values = to_vector();
    const std::size_t shown = std::min<std::size_t>(values.size(), 8);
    for (std::size_t i = 0; i < shown; ++i) s << (i ? ", " : "") << std::setprecision(6) << values[i];
    if (values.size() > shown) s << ", ...";
    s << "])";
    return s.str();
}

Tensor operator+(const Tensor& a, const Tensor& b) { return add(a, b); }
Tensor operator-(const Tensor& a, const Tensor& b) { return subtract(a, b); }
Tensor operator*(const Tensor& a, const Tensor& b) { return multiply(a, b); }
Tensor operator/(const Tensor& a, const Tensor& b) { return divide(a, b); }
Tensor operator-(const Tensor& v) { return negate(v); }
Tensor operator+(const Tensor& a, float b) { return a + Tensor::scalar(b, false, a.device()); }
Tensor operator-(const Tensor& a, float b) { return a - Tensor::scalar(b, false, a.device()); }
Tensor operator*(const Tensor& a, float b) { return a * Tensor::scalar(b, false, a.device()); }
Tensor operator/(const Tensor& a, float b) { return a / Tensor::scalar(b, false, a.device()); }
Tensor operator+(float a, const Tensor& b) { return Tensor::scalar(a, false, b.device()) + b; }
Tensor operator-(float a, const Tensor& b) { return Tensor::scalar(a, false, b.device()) - b; }
Tensor operator*(float a, const Tensor& b) { return Tensor::scalar(a, false, b.device()) * b; }
Tensor operator/(float a, const Tensor& b) { return Tensor::scalar(a, false, b.device()) / b; }

}  // namespace vectorcore
