#pragma once
// Graph and tensor internals (API of include/vectorcore/detail/tensor_impl.hpp).
#include "vectorcore/shape.hpp"
#include "vectorcore/storage.hpp"
#include "vectorcore/tensor.hpp"

#include <functional>
#include <memory>
#include <optional>
#include <vector>

namespace vectorcore::detail {

struct TensorImpl;

// A node owns its parents (never its children), so graphs have no cycles.
struct GradFn {
    std::vector<std::shared_ptr<TensorImpl>> parents;
    std::function<std::vector<Tensor>(const Tensor&)> backward;
    // Set by relu(): a tensor whose positive entries are those of the ReLU's
    // input (the input's version is checked). Lets the engine offer the ReLU
    // mask to the node that produces this node's upstream gradient (see
    // ReluMaskOffer).
    std::function<Tensor()> relu_mask;
};

// The engine's offer to the backward rule it is about to run: parent 0 of
// that node is a ReLU output with no other consumer in the graph and no
// retained gradient, so the rule may return parent 0's gradient already
// multiplied by [relu_mask() > 0] (the ReLU rule's own arithmetic) and set
// `taken`; the engine then passes that gradient through the ReLU node as is.
struct ReluMaskOffer {
    std::function<Tensor()> relu_mask;
    bool taken = false;
};
// The offer in effect on this thread, or null.
ReluMaskOffer* relu_mask_offer();
void set_relu_mask_offer(ReluMaskOffer* offer);

struct TensorImpl {
    std::shared_ptr<Storage> storage;
    Shape shape;
    Strides strides;
    std::size_t offset{0};
    DType dtype{DType::Float32};
    bool requires_grad{false};
    bool leaf{true};
    bool retains_grad{false};
    std::shared_ptr<GradFn> grad_fn;
    std::shared_ptr<TensorImpl> grad;
};

// A tensor saved for a backward rule with its storage version; unpack()
// throws std::runtime_error if the storage was modified in place since.
class SavedTensor {
public:
    explicit SavedTensor(const Tensor& value);
    [[nodiscard]] Tensor unpack() const;
    // The tensor if its storage is unchanged since it was saved, else nothing.
    [[nodiscard]] std::optional<Tensor> unpack_if_unchanged() const;
private:
    Tensor tensor_;
    std::uint64_t version_;
};

Tensor from_impl(std::shared_ptr<TensorImpl> impl);
Tensor make_tensor(std::shared_ptr<Storage> storage, Shape shape, bool requires_grad = false);
void attach_grad_fn(Tensor& output, const std::vector<Tensor>& parents,
                    std::function<std::vector<Tensor>(const Tensor&)> backward);
Tensor sum_to_shape(const Tensor& gradient, const Shape& target_shape);
Tensor broadcast_to(const Tensor& value, const Shape& target_shape);

}  // namespace vectorcore::detail
