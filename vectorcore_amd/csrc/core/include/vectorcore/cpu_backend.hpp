#pragma once
// Host kernels of the `cpu` device (API of include/vectorcore/cpu_backend.hpp).
#include "vectorcore/shape.hpp"

#include <cstddef>

namespace vectorcore::cpu {

enum class BinaryOp { Add, Subtract, Multiply, Divide };
enum class UnaryOp { Negate, Relu, Sigmoid, ReluGradient, Exp, Log };
enum class ReduceOp { Sum, Max, Argmax };

void binary(const float* a, const Shape& a_shape, const Strides& a_strides, const float* b, const Shape& b_shape,
            const Strides& b_strides, float* out, const Shape& out_shape, BinaryOp operation);
void unary(const float* input, float* output, std::size_t count, UnaryOp operation);
// out (m x n) = op(a) @ op(b), row-major; trans_a: a stored (k x m); trans_b: b stored (n x k).
void matmul(const float* a, const float* b, float* out, std::size_t m, std::size_t k, std::size_t n,
            bool trans_a = false, bool trans_b = false);
void transpose(const float* input, float* output, std::size_t batch, std::size_t rows, std::size_t cols);
float sum(const float* input, std::size_t count);
// [outer, length, inner] -> [outer, inner]; argmax writes the first winning index as a float.
void reduce_axis(const float* input, float* output, std::size_t outer, std::size_t length, std::size_t inner,
                 ReduceOp operation);
// Inverse of argmax: output is zero except output[o, indices[o, i], i] = values[o, i].
void scatter_axis(const float* values, const float* indices, float* output, std::size_t outer, std::size_t length,
                  std::size_t inner);

}  // namespace vectorcore::cpu
