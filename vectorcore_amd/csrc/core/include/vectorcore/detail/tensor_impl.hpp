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
    // GradientOffer).
    std::function<Tensor()> relu_mask;
    // Set by add() when one operand is a row bias ([n] or [1, n]) added to a
    // 2-D [m, n] operand: its index. The bias's gradient is then the column
    // sum of this node's upstream gradient (sum_to_shape).
    int row_bias_operand = -1;
};

// The engine's offer to the backward rule it is about to run, about the
// gradient the rule returns for its parent 0. Either part may be absent.
// - relu_mask: parent 0 is a ReLU output with no other consumer in the graph
//   and no retained gradient, so the rule may return parent 0's gradient
//   already multiplied by [relu_mask() > 0] (the ReLU rule's own arithmetic)
//   and set `taken`; the engine then passes that gradient through the ReLU
//   node as is.
// - column_sum_wanted: the gradient the rule returns for parent 0 will reach a
//   row-bias add (row_bias_operand) with no other consumer whose bias needs a
//   gradient, unchanged (parent 0 is that add, or the ReLU above it whose mask
//   is offered): the add's rule will take its column sum. A rule that can
//   produce the sum on the way may leave it with the gradient's storage.
struct GradientOffer {
    std::function<Tensor()> relu_mask;
    bool column_sum_wanted = false;
    bool taken = false;
};
// The offer in effect on this thread, or null.
GradientOffer* gradient_offer();
void set_gradient_offer(GradientOffer* offer);

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
