#pragma once
// Layers, losses and the optimizer step (API of include/vectorcore/nn.hpp).
#include "vectorcore/tensor.hpp"

#include <cstdint>
#include <vector>

namespace vectorcore::nn {

class Linear {
public:
    Linear(std::size_t in_features, std::size_t out_features, std::uint64_t seed = 0);
    Tensor operator()(const Tensor& input) const;
    std::vector<Tensor*> parameters();
    Tensor weight;  // [in_features, out_features]
    Tensor bias;    // [out_features]
};

Tensor mse_loss(const Tensor& prediction, const Tensor& target);
// Mean negative log-likelihood of integer class targets under softmax(logits).
Tensor cross_entropy(const Tensor& logits, const std::vector<std::size_t>& targets);
// In-place p -= lr * grad on every parameter that has a gradient; bumps versions.
void sgd_step(const std::vector<Tensor*>& parameters, float learning_rate);
void zero_grad(const std::vector<Tensor*>& parameters);

}  // namespace vectorcore::nn
