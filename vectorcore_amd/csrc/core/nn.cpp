#include "vectorcore/nn.hpp"

#include "vectorcore/autograd.hpp"
#include "vectorcore/detail/tensor_impl.hpp"
#include "vectorcore/hip_backend.hpp"
#include "vectorcore/ops.hpp"

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>

namespace vectorcore::nn {

Linear::Linear(std::size_t in_features, std::size_t out_features, std::uint64_t seed)
    : weight(Tensor::randn({in_features, out_features}, true, seed) / std::sqrt(static_cast<float>(in_features))),
      bias(Tensor::zeros({out_features}, true)) {
    // The scaled weight is a graph node; make it a leaf parameter again.
    weight = weight.detach();
    weight.set_requires_grad(true);
}

Tensor Linear::operator()(const Tensor& input) const { return input.matmul(weight) + bias; }
std::vector<Tensor*> Linear::parameters() { return {&weight, &bias}; }

Tensor mse_loss(const Tensor& prediction, const Tensor& target) {
    const Tensor error = prediction - target;
    return (error * error).mean();
}

namespace {

void check_targets(const Tensor& logits, const std::vector<std::size_t>& targets) {
    if (logits.ndim() != 2)
        throw std::invalid_argument("cross_entropy expects [batch, classes] logits, got " + shape_string(logits.shape()));
    const std::size_t batch = logits.shape()[0], classes = logits.shape()[1];
    if (targets.size() != batch)
        throw std::invalid_argument("cross_entropy received " + std::to_string(targets.size()) + " targets for a batch of " +
                                    std::to_string(batch));
    if (batch == 0) throw std::invalid_argument("cross_entropy of an empty batch is undefined");
    for (std::size_t t : targets)
        if (t >= classes)
            throw std::out_of_range("target class " + std::to_string(t) + " is out of range for " +
                                    std::to_string(classes) + " classes");
}

// One loss node on the device (forward and backward kernels of the whole
// composition); see the hip path in cross_entropy below.
Tensor cross_entropy_hip(const Tensor& logits, const std::vector<std::size_t>& targets) {
    auto& hip = HipBackend::instance();
    const std::size_t rows = logits.shape()[0], classes = logits.shape()[1];
    if (classes > 0x7fffffffU) throw std::overflow_error("cross_entropy: too many classes for int32 targets");
    std::shared_ptr<Storage> dev_targets = hip.upload_targets(targets);
    auto [loss_storage, stats] =
        hip.cross_entropy_forward(*logits.impl()->storage, logits.impl()->offset, *dev_targets, rows, classes);
    Tensor loss = detail::make_tensor(std::move(loss_storage), {}, false);
    const detail::SavedTensor saved(logits);
    std::shared_ptr<Storage> row_stats = std::move(stats);
    detail::attach_grad_fn(loss, {logits}, [saved, dev_targets, row_stats, rows, classes](const Tensor& g) {
        const Tensor x = saved.unpack();
        // When the logits are h @ W + b, the backward kernel also leaves the
        // column sums that b's add rule takes next (see GradientOffer).
        const detail::GradientOffer* offer = detail::gradient_offer();
        const bool column_sum = offer && offer->column_sum_wanted && !offer->relu_mask;
        auto d = HipBackend::instance().cross_entropy_backward(*x.impl()->storage, x.impl()->offset, *dev_targets,
                                                               *row_stats, *g.impl()->storage, g.impl()->offset, rows,
                                                               classes, column_sum);
        return std::vector<Tensor>{detail::make_tensor(std::move(d), {rows, classes}, false)};
    });
    return loss;
}

}  // namespace

// -(log_softmax(logits, 1) * one_hot).sum() / batch. On the cpu device this is
// composed from tensor ops with a host one-hot mask (src/nn.cpp:31-53). On hip
// it is one loss node whose forward and backward kernels evaluate the same
// composition per row, with N int32 class indices instead of an [N, C] mask.
Tensor cross_entropy(const Tensor& logits, const std::vector<std::size_t>& targets) {
    check_targets(logits, targets);
    if (logits.device() == Device::hip()) return cross_entropy_hip(logits, targets);
    const std::size_t batch = logits.shape()[0], classes = logits.shape()[1];
    std::vector<float> one_hot(batch * classes, 0.0F);
    for (std::size_t r = 0; r < batch; ++r) one_hot[r * classes + targets[r]] = 1.0F;
    const Tensor mask(std::move(one_hot), {batch, classes}, false, logits.device());
    return -(logits.log_softmax(1) * mask).sum() / static_cast<float>(batch);
}

void sgd_step(const std::vector<Tensor*>& parameters, float learning_rate) {
    NoGradGuard guard;
    // hip parameters are updated in batches (one launch for up to 16), in
    // parameter order: a batch is flushed before anything that the reference's
    // one-at-a-time loop would order after it (an error, a cpu parameter, a
    // parameter sharing a batched storage).
    std::vector<HipBackend::AxpyItem> batch;
    std::vector<Storage*> touched;        // targets in the batch
    std::vector<const Storage*> read;     // sources in the batch
    const auto contains = [](const auto& v, const Storage* s) { return std::find(v.begin(), v.end(), s) != v.end(); };
    const auto flush = [&] {
        if (batch.empty()) return;
        HipBackend::instance().axpy_batch(batch, -learning_rate);
        for (Storage* s : touched) s->bump_version();  // an in-place update, like mutable_data()
        batch.clear();
        touched.clear();
        read.clear();
    };
    for (Tensor* p : parameters) {
        if (!p || !p->has_grad()) continue;
        const Tensor g = p->grad();
        if (g.shape() != p->shape() || g.device() != p->device()) {
            flush();
            throw std::invalid_argument("parameter gradient shape or device does not match");
        }
        if (p->device() == Device::hip()) {
            Storage* storage = p->impl()->storage.get();
            const Storage* source = g.impl()->storage.get();
            if (contains(touched, storage) || contains(read, storage) || contains(touched, source)) flush();
            batch.push_back({storage, p->impl()->offset, source, g.impl()->offset, p->numel()});
            touched.push_back(storage);
            read.push_back(source);
            continue;
        }
        flush();
        if (p->device() != Device::cpu()) throw std::runtime_error("Metal is unavailable: VectorCore was built without Apple Metal");
        const auto gv = g.to_vector();
        float* values = p->mutable_data();
        for (std::size_t i = 0; i < p->numel(); ++i) values[i] -= learning_rate * gv[i];
    }
    flush();
}

void zero_grad(const std::vector<Tensor*>& parameters) {
    for (Tensor* p : parameters)
        if (p) p->zero_grad();
}

}  // namespace vectorcore::nn
