// Differentiable operations and their device dispatch.
//
// Each op computes its forward on the operands' device and records a backward
// rule with the semantics of src/ops.cpp. The `hip` arm of a backward rule may
// call one fused kernel where the CPU arm composes several ops (activation
// gradients, the division gradient, the batch-broadcast matmul gradient);
// graph structure, saved tensors and version checks are the same on both.
#include "vectorcore/ops.hpp"

#include "vectorcore/autograd.hpp"
#include "vectorcore/cpu_backend.hpp"
#include "vectorcore/detail/tensor_impl.hpp"
#include "vectorcore/hip_backend.hpp"
#include "vectorcore/storage.hpp"

#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace vectorcore {

namespace {

[[noreturn]] void metal_unavailable() {
    throw std::runtime_error("Metal is unavailable: VectorCore was built without Apple Metal");
}

// A rule's two gradients as one vector. Both are complete objects before the
// vector is built, so when computing the second throws (a version check),
// the first is destroyed; a brace-initialised vector built from the two
// expressions leaks the first under GCC 11, which does not destroy the
// already-built elements of a partly built initializer list.
std::vector<Tensor> two_grads(Tensor first, Tensor second) {
    std::vector<Tensor> out;
    out.reserve(2);
    out.push_back(std::move(first));
    out.push_back(std::move(second));
    return out;
}

HipBackend& hip() { return HipBackend::instance(); }
const Storage& st(const Tensor& t) { return *t.impl()->storage; }
std::size_t off(const Tensor& t) { return t.impl()->offset; }

void require_same_device(const Tensor& a, const Tensor& b) {
    if (a.device() != b.device())
        throw std::invalid_argument("tensor device mismatch: " + a.device().str() + " vs " + b.device().str());
}

Tensor binary_forward(const Tensor& a, const Tensor& b, cpu::BinaryOp op) {
    require_same_device(a, b);
    const Shape out_shape = broadcast_shape(a.shape(), b.shape());
    std::shared_ptr<Storage> s;
    switch (a.device().type) {
        case DeviceType::CPU:
            s = make_cpu_storage(numel(out_shape));
            cpu::binary(a.data(), a.shape(), a.strides(), b.data(), b.shape(), b.strides(), s->mutable_data(), out_shape,
                        op);
            break;
        case DeviceType::HIP:
            s = hip().binary(st(a), off(a), a.shape(), a.strides(), st(b), off(b), b.shape(), b.strides(), out_shape, op);
            break;
        case DeviceType::METAL: metal_unavailable();
    }
    return detail::make_tensor(std::move(s), out_shape, false);
}

Tensor unary_forward(const Tensor& v, cpu::UnaryOp op) {
    std::shared_ptr<Storage> s;
    switch (v.device().type) {
        case DeviceType::CPU:
            s = make_cpu_storage(v.numel());
            cpu::unary(v.data(), s->mutable_data(), v.numel(), op);
            break;
        case DeviceType::HIP: s = hip().unary(st(v), off(v), v.numel(), op); break;
        case DeviceType::METAL: metal_unavailable();
    }
    return detail::make_tensor(std::move(s), v.shape(), false);
}

// Fused activation gradient on hip; the reference's composition on cpu.
Tensor activation_grad(HipBackend::Activation kind, const Tensor& g, const Tensor& saved) {
    if (g.device() == Device::hip() && g.shape() == saved.shape()) {
        return detail::make_tensor(hip().activation_backward(kind, st(g), off(g), st(saved), off(saved), g.numel()),
                                   g.shape(), false);
    }
    switch (kind) {
        case HipBackend::Activation::Relu: return g * unary_forward(saved, cpu::UnaryOp::ReluGradient);
        case HipBackend::Activation::Sigmoid: return g * saved * (1.0F - saved);
        case HipBackend::Activation::Exp: return g * saved;
        case HipBackend::Activation::Log: return g / saved;
    }
    throw std::logic_error("unknown activation");
}

struct AxisSplit {
    std::size_t axis, outer, length, inner;
    Shape kept;     // reduced axis set to 1
    Shape removed;  // reduced axis dropped
};

AxisSplit split_axis(const Shape& shape, std::int64_t axis) {
    const auto rank = static_cast<std::int64_t>(shape.size());
    if (rank == 0) throw std::invalid_argument("cannot reduce a scalar along an axis");
    if (axis < -rank || axis >= rank)
        throw std::out_of_range("axis " + std::to_string(axis) + " is out of range for shape " + shape_string(shape));
    AxisSplit s{};
    s.axis = static_cast<std::size_t>(axis < 0 ? axis + rank : axis);
    s.outer = numel(Shape(shape.begin(), shape.begin() + static_cast<std::ptrdiff_t>(s.axis)));
    s.length = shape[s.axis];
    s.inner = numel(Shape(shape.begin() + static_cast<std::ptrdiff_t>(s.axis) + 1, shape.end()));
    s.kept = shape;
    s.kept[s.axis] = 1;
    s.removed = shape;
    s.removed.erase(s.removed.begin() + static_cast<std::ptrdiff_t>(s.axis));
    return s;
}

std::shared_ptr<Storage> reduce_storage(const Tensor& v, const AxisSplit& s, cpu::ReduceOp op) {
    switch (v.device().type) {
        case DeviceType::CPU: {
            auto out = make_cpu_storage(s.outer * s.inner);
            cpu::reduce_axis(v.data(), out->mutable_data(), s.outer, s.length, s.inner, op);
            return out;
        }
        case DeviceType::HIP: return hip().reduce_axis(st(v), off(v), s.outer, s.length, s.inner, op);
        case DeviceType::METAL: metal_unavailable();
    }
    throw std::logic_error("unknown device");
}

// Batch layout of a matmul: per output batch z, the element offsets of the A
// and B matrices it reads (broadcast batch axes reuse one matrix).
struct MatmulPlan {
    std::size_t m, k, n, batch;
    Shape out_batch, a_batch, b_batch;
    std::vector<std::size_t> a_offsets, b_offsets;
};

MatmulPlan plan_matmul(const Tensor& a, const Tensor& b, bool trans_a, bool trans_b) {
    if (a.ndim() < 2 || b.ndim() < 2)
        throw std::invalid_argument("matmul requires tensors of rank 2 or more, got " + shape_string(a.shape()) + " and " +
                                    shape_string(b.shape()));
    const Shape& as = a.shape();
    const Shape& bs = b.shape();
    const std::size_t ar = as[as.size() - 2], ac = as.back(), br = bs[bs.size() - 2], bc = bs.back();
    MatmulPlan p{};
    p.m = trans_a ? ac : ar;
    p.k = trans_a ? ar : ac;
    p.n = trans_b ? br : bc;
    if ((trans_b ? bc : br) != p.k)
        throw std::invalid_argument("matmul shape mismatch: " + shape_string(as) + " and " + shape_string(bs));
    p.a_batch = Shape(as.begin(), as.end() - 2);
    p.b_batch = Shape(bs.begin(), bs.end() - 2);
    try {
        p.out_batch = broadcast_shape(p.a_batch, p.b_batch);
    } catch (const std::invalid_argument&) {
        throw std::invalid_argument("matmul batch dimensions do not broadcast: " + shape_string(as) + " and " +
                                    shape_string(bs));
    }
    p.batch = numel(p.out_batch);
    const Strides sa = contiguous_strides(p.a_batch), sb = contiguous_strides(p.b_batch);
    const std::size_t rank = p.out_batch.size();
    p.a_offsets.resize(p.batch);
    p.b_offsets.resize(p.batch);
    for (std::size_t z = 0; z < p.batch; ++z) {
        std::size_t rem = z, ia = 0, ib = 0;
        for (std::size_t ax = rank; ax-- > 0;) {
            const std::size_t c = rem % p.out_batch[ax];
            rem /= p.out_batch[ax];
            if (ax + p.a_batch.size() >= rank) {
                const std::size_t i = ax + p.a_batch.size() - rank;
                if (p.a_batch[i] != 1) ia += c * sa[i];
            }
            if (ax + p.b_batch.size() >= rank) {
                const std::size_t i = ax + p.b_batch.size() - rank;
                if (p.b_batch[i] != 1) ib += c * sb[i];
            }
        }
        p.a_offsets[z] = ia * p.m * p.k;
        p.b_offsets[z] = ib * p.k * p.n;
    }
    return p;
}

// op(A) @ op(B) without a gradient rule (transposes read in place).
Tensor matmul_kernel(const Tensor& a, const Tensor& b, bool trans_a, bool trans_b,
                     const Tensor* relu_mask = nullptr, bool column_sum = false) {
    require_same_device(a, b);
    const MatmulPlan p = plan_matmul(a, b, trans_a, trans_b);
    if (relu_mask) {  // hip only: the product times [relu_mask > 0], relu_mask shaped like the product
        auto s = hip().matmul_relu_mask(st(a), off(a), st(b), off(b), p.m, p.k, p.n, p.a_offsets, p.b_offsets,
                                        trans_a, trans_b, st(*relu_mask), off(*relu_mask),
                                        column_sum && p.batch == 1);
        Shape out_shape = p.out_batch;
        out_shape.push_back(p.m);
        out_shape.push_back(p.n);
        return detail::make_tensor(std::move(s), out_shape, false);
    }
    std::shared_ptr<Storage> s;
    switch (a.device().type) {
        case DeviceType::CPU: {
            s = make_cpu_storage(p.batch * p.m * p.n);
            float* out = s->mutable_data();
            for (std::size_t z = 0; z < p.batch; ++z)
                cpu::matmul(a.data() + p.a_offsets[z], b.data() + p.b_offsets[z], out + z * p.m * p.n, p.m, p.k, p.n,
                            trans_a, trans_b);
            break;
        }
        case DeviceType::HIP:
            s = hip().matmul(st(a), off(a), st(b), off(b), p.m, p.k, p.n, p.a_offsets, p.b_offsets, trans_a, trans_b);
            break;
        case DeviceType::METAL: metal_unavailable();
    }
    Shape out_shape = p.out_batch;
    out_shape.push_back(p.m);
    out_shape.push_back(p.n);
    return detail::make_tensor(std::move(s), out_shape, false);
}

// Element stride between consecutive output batches of an operand whose batch
// axes are either all present (== out_batch) or all broadcast; -1 otherwise.
std::int64_t uniform_batch_stride(const Shape& batch_axes, const Shape& out_batch, std::size_t matrix_elems) {
    if (numel(batch_axes) == 1) return 0;
    Shape padded(out_batch.size() - batch_axes.size(), 1);
    padded.insert(padded.end(), batch_axes.begin(), batch_axes.end());
    return padded == out_batch ? static_cast<std::int64_t>(matrix_elems) : -1;
}

}  // namespace

// --- elementwise -------------------------------------------------------------

namespace {

// hip: a row-bias add applied to a product not computed yet joins the
// product's epilogue (either operand order: fp32 a + b == b + a).
std::optional<Tensor> add_bias_deferred(const Tensor& a, const Tensor& b) {
    if (a.device() != Device::hip() || b.device() != Device::hip()) return std::nullopt;
    for (int order = 0; order < 2; ++order) {
        const Tensor& product = order == 0 ? a : b;
        const Tensor& bias = order == 0 ? b : a;
        auto s = hip().add_bias_deferred(st(product), off(product), product.shape(), product.strides(),
                                         bias.impl()->storage, off(bias), bias.shape(), bias.strides());
        if (s) return detail::make_tensor(std::move(s), product.shape(), false);
    }
    return std::nullopt;
}

}  // namespace

Tensor add(const Tensor& a, const Tensor& b) {
    std::optional<Tensor> fused = add_bias_deferred(a, b);
    auto out = fused ? *fused : binary_forward(a, b, cpu::BinaryOp::Add);
    const Shape as = a.shape(), bs = b.shape();
    const bool na = a.requires_grad(), nb = b.requires_grad();
    detail::attach_grad_fn(out, {a, b}, [=](const Tensor& g) {
        return two_grads(na ? detail::sum_to_shape(g, as) : Tensor(), nb ? detail::sum_to_shape(g, bs) : Tensor());
    });
    if (out.impl()->grad_fn) {  // a row bias added to a matrix: its gradient is a column sum
        const auto row_bias = [](const Shape& matrix, const Shape& bias) {
            return matrix.size() == 2 && (bias == Shape{matrix[1]} || bias == Shape{1, matrix[1]});
        };
        if (row_bias(as, bs)) out.impl()->grad_fn->row_bias_operand = 1;
        else if (row_bias(bs, as)) out.impl()->grad_fn->row_bias_operand = 0;
    }
    return out;
}

Tensor subtract(const Tensor& a, const Tensor& b) {
    auto out = binary_forward(a, b, cpu::BinaryOp::Subtract);
    const Shape as = a.shape(), bs = b.shape();
    const bool na = a.requires_grad(), nb = b.requires_grad();
    detail::attach_grad_fn(out, {a, b}, [=](const Tensor& g) {
        return two_grads(na ? detail::sum_to_shape(g, as) : Tensor(), nb ? detail::sum_to_shape(-g, bs) : Tensor());
    });
    return out;
}

Tensor multiply(const Tensor& a, const Tensor& b) {
    auto out = binary_forward(a, b, cpu::BinaryOp::Multiply);
    const Shape as = a.shape(), bs = b.shape();
    const bool na = a.requires_grad(), nb = b.requires_grad();
    const detail::SavedTensor sa(a), sb(b);
    detail::attach_grad_fn(out, {a, b}, [=](const Tensor& g) {
        return two_grads(na ? detail::sum_to_shape(g * sb.unpack(), as) : Tensor(),
                                   nb ? detail::sum_to_shape(g * sa.unpack(), bs) : Tensor());
    });
    return out;
}

Tensor divide(const Tensor& a, const Tensor& b) {
    auto out = binary_forward(a, b, cpu::BinaryOp::Divide);
    const Shape as = a.shape(), bs = b.shape();
    const bool na = a.requires_grad(), nb = b.requires_grad();
    const detail::SavedTensor sa(a), sb(b);
    detail::attach_grad_fn(out, {a, b}, [=](const Tensor& g) {
        std::vector<Tensor> grads{Tensor(), Tensor()};
        const Tensor bv = sb.unpack();
        if (g.device() == Device::hip()) {
            // One pass over the output shape for both quotients' gradients.
            const Tensor av = sa.unpack();
            auto [ga, gb] = hip().divide_backward(st(g), off(g), st(av), off(av), av.shape(), av.strides(), st(bv), off(bv),
                                                  bv.shape(), bv.strides(), g.shape(), na, nb);
            if (na) grads[0] = detail::sum_to_shape(detail::make_tensor(ga, g.shape()), as);
            if (nb) grads[1] = detail::sum_to_shape(detail::make_tensor(gb, g.shape()), bs);
            return grads;
        }
        if (na) grads[0] = detail::sum_to_shape(g / bv, as);
        if (nb) grads[1] = detail::sum_to_shape(-(g * sa.unpack()) / (bv * bv), bs);
        return grads;
    });
    return out;
}

Tensor negate(const Tensor& v) {
    auto out = unary_forward(v, cpu::UnaryOp::Negate);
    detail::attach_grad_fn(out, {v}, [](const Tensor& g) { return std::vector<Tensor>{-g}; });
    return out;
}

// --- matrix products -------------------------------------------------------------

namespace {

// hip: a 2-D product is recorded and computed on first use, so that a
// following bias add and ReLU can join its epilogue (HipBackend::matmul_deferred).
std::optional<Tensor> matmul_deferred(const Tensor& a, const Tensor& b) {
    if (a.device() != Device::hip() || b.device() != Device::hip() || a.ndim() != 2 || b.ndim() != 2)
        return std::nullopt;
    if (a.strides() != contiguous_strides(a.shape()) || b.strides() != contiguous_strides(b.shape()))
        return std::nullopt;
    const MatmulPlan p = plan_matmul(a, b, false, false);
    auto s = hip().matmul_deferred(a.impl()->storage, off(a), b.impl()->storage, off(b), p.m, p.k, p.n);
    if (!s) return std::nullopt;
    return detail::make_tensor(std::move(s), Shape{p.m, p.n}, false);
}

}  // namespace

Tensor matmul(const Tensor& a, const Tensor& b) {
    std::optional<Tensor> deferred = matmul_deferred(a, b);
    auto out = deferred ? *deferred : matmul_kernel(a, b, false, false);
    const detail::SavedTensor sa(a), sb(b);
    const Shape as = a.shape(), bs = b.shape();
    const bool na = a.requires_grad(), nb = b.requires_grad();
    detail::attach_grad_fn(out, {a, b}, [=](const Tensor& g) {
        // dA = dY @ B^T, dB = A^T @ dY; a batch-broadcast operand receives the
        // sum over the batches it was reused for.
        std::vector<Tensor> grads{Tensor(), Tensor()};
        const Tensor av = sa.unpack(), bv = sb.unpack();
        if (g.device() == Device::hip()) {
            const MatmulPlan p = plan_matmul(av, bv, false, false);
            const std::int64_t a_step = uniform_batch_stride(p.a_batch, p.out_batch, p.m * p.k);
            const std::int64_t b_step = uniform_batch_stride(p.b_batch, p.out_batch, p.k * p.n);
            if (na && p.batch > 1 && numel(p.a_batch) == 1 && b_step >= 0) {
                // dA = sum_z dY_z @ B_z^T in one batch-reduced product.
                auto s = hip().matmul_reduce(st(g), off(g), st(bv), off(bv), p.m, p.n, p.k, p.batch, p.m * p.n,
                                             static_cast<std::size_t>(b_step), false, true);
                grads[0] = detail::make_tensor(std::move(s), as);
            } else if (na) {
                // The engine may offer A's ReLU mask (A = relu(x) feeding only
                // this product): dA * [x > 0] comes out of the same kernel.
                detail::GradientOffer* offer = detail::gradient_offer();
                Shape product = p.out_batch;
                product.push_back(p.m);
                product.push_back(p.k);
                std::optional<Tensor> relu_mask;
                if (offer && offer->relu_mask && product == as) {
                    relu_mask = offer->relu_mask();
                    if (relu_mask->device() != Device::hip() || relu_mask->shape() != as ||
                        relu_mask->strides() != contiguous_strides(as))
                        relu_mask.reset();
                }
                if (relu_mask) {
                    // When the ReLU's input is a bias add, the product's epilogue
                    // also leaves the column sums that the add rule will ask for.
                    grads[0] = matmul_kernel(g, bv, false, true, &*relu_mask, offer->column_sum_wanted);
                    offer->taken = true;
                } else {
                    grads[0] = detail::sum_to_shape(matmul_kernel(g, bv, false, true), as);
                }
            }
            if (nb && p.batch > 1 && numel(p.b_batch) == 1 && a_step >= 0) {
                // dB = sum_z A_z^T @ dY_z.
                auto s = hip().matmul_reduce(st(av), off(av), st(g), off(g), p.k, p.m, p.n, p.batch,
                                             static_cast<std::size_t>(a_step), p.m * p.n, true, false);
                grads[1] = detail::make_tensor(std::move(s), bs);
            } else if (nb) {
                grads[1] = detail::sum_to_shape(matmul_kernel(av, g, true, false), bs);
            }
            return grads;
        }
        if (na) grads[0] = detail::sum_to_shape(matmul_kernel(g, bv, false, true), as);
        if (nb) grads[1] = detail::sum_to_shape(matmul_kernel(av, g, true, false), bs);
        return grads;
    });
    return out;
}

Tensor transpose(const Tensor& v) {
    if (v.ndim() < 2) throw std::invalid_argument("transpose requires a tensor of rank 2 or more");
    const Shape& shape = v.shape();
    const std::size_t rows = shape[shape.size() - 2], cols = shape.back();
    const std::size_t batch = numel(Shape(shape.begin(), shape.end() - 2));
    std::shared_ptr<Storage> s;
    switch (v.device().type) {
        case DeviceType::CPU:
            s = make_cpu_storage(v.numel());
            cpu::transpose(v.data(), s->mutable_data(), batch, rows, cols);
            break;
        case DeviceType::HIP: s = hip().transpose_last2(st(v), off(v), batch, rows, cols); break;
        case DeviceType::METAL: metal_unavailable();
    }
    Shape out_shape = shape;
    std::swap(out_shape[out_shape.size() - 2], out_shape.back());
    auto out = detail::make_tensor(std::move(s), out_shape, false);
    detail::attach_grad_fn(out, {v}, [](const Tensor& g) { return std::vector<Tensor>{g.transpose()}; });
    return out;
}

// --- reductions --------------------------------------------------------------------

Tensor sum(const Tensor& v) {
    std::shared_ptr<Storage> s;
    switch (v.device().type) {
        case DeviceType::CPU: {
            const float r = cpu::sum(v.data(), v.numel());
            s = make_cpu_storage(&r, 1);
            break;
        }
        case DeviceType::HIP: s = hip().reduce_sum(st(v), off(v), v.numel()); break;
        case DeviceType::METAL: metal_unavailable();
    }
    auto out = detail::make_tensor(std::move(s), {}, false);
    const Shape in_shape = v.shape();
    detail::attach_grad_fn(out, {v}, [in_shape](const Tensor& g) {
        return std::vector<Tensor>{detail::broadcast_to(g, in_shape)};
    });
    return out;
}

Tensor sum(const Tensor& v, std::int64_t axis, bool keepdim) {
    const AxisSplit s = split_axis(v.shape(), axis);
    auto out = detail::make_tensor(reduce_storage(v, s, cpu::ReduceOp::Sum), keepdim ? s.kept : s.removed, false);
    const Shape in_shape = v.shape(), kept = s.kept;
    detail::attach_grad_fn(out, {v}, [in_shape, kept](const Tensor& g) {
        return std::vector<Tensor>{detail::broadcast_to(g.reshape(kept), in_shape)};
    });
    return out;
}

Tensor mean(const Tensor& v, std::int64_t axis, bool keepdim) {
    const AxisSplit s = split_axis(v.shape(), axis);
    if (s.length == 0) throw std::invalid_argument("mean over an empty axis is undefined");
    return sum(v, axis, keepdim) / static_cast<float>(s.length);
}

Tensor mean(const Tensor& v) {
    if (v.numel() == 0) throw std::invalid_argument("mean of an empty tensor is undefined");
    return v.sum() / static_cast<float>(v.numel());
}

Tensor max(const Tensor& v, std::int64_t axis, bool keepdim) {
    const AxisSplit s = split_axis(v.shape(), axis);
    const Shape out_shape = keepdim ? s.kept : s.removed;
    auto out = detail::make_tensor(reduce_storage(v, s, cpu::ReduceOp::Max), out_shape, false);
    if (!grad_enabled() || !v.requires_grad()) return out;
    // The gradient goes to the first maximal element along the axis.
    const Tensor indices = detail::make_tensor(reduce_storage(v, s, cpu::ReduceOp::Argmax), out_shape, false);
    const Shape in_shape = v.shape();
    detail::attach_grad_fn(out, {v}, [indices, s, in_shape](const Tensor& g) {
        std::shared_ptr<Storage> r;
        switch (g.device().type) {
            case DeviceType::CPU:
                r = make_cpu_storage(numel(in_shape));
                cpu::scatter_axis(g.data(), indices.data(), r->mutable_data(), s.outer, s.length, s.inner);
                break;
            case DeviceType::HIP:
                r = hip().scatter_axis(st(g), off(g), st(indices), off(indices), s.outer, s.length, s.inner);
                break;
            case DeviceType::METAL: metal_unavailable();
        }
        return std::vector<Tensor>{detail::make_tensor(std::move(r), in_shape, false)};
    });
    return out;
}

Tensor max(const Tensor& v) {
    if (v.numel() == 0) throw std::invalid_argument("max of an empty tensor is undefined");
    return max(v.flatten(), 0, false);
}

Tensor argmax(const Tensor& v, std::int64_t axis, bool keepdim) {
    const AxisSplit s = split_axis(v.shape(), axis);
    return detail::make_tensor(reduce_storage(v, s, cpu::ReduceOp::Argmax), keepdim ? s.kept : s.removed, false);
}

// --- activations ---------------------------------------------------------------------

Tensor exp(const Tensor& v) {
    auto out = unary_forward(v, cpu::UnaryOp::Exp);
    const detail::SavedTensor saved(out);
    detail::attach_grad_fn(out, {v}, [saved](const Tensor& g) {
        return std::vector<Tensor>{activation_grad(HipBackend::Activation::Exp, g, saved.unpack())};
    });
    return out;
}

Tensor log(const Tensor& v) {
    auto out = unary_forward(v, cpu::UnaryOp::Log);
    const detail::SavedTensor saved(v);
    detail::attach_grad_fn(out, {v}, [saved](const Tensor& g) {
        return std::vector<Tensor>{activation_grad(HipBackend::Activation::Log, g, saved.unpack())};
    });
    return out;
}

Tensor relu(const Tensor& v) {
    std::shared_ptr<Storage> fused;
    if (v.device() == Device::hip()) fused = hip().relu_deferred(st(v), off(v), v.numel());
    auto out = fused ? detail::make_tensor(std::move(fused), v.shape(), false) : unary_forward(v, cpu::UnaryOp::Relu);
    // The rule's mask [input > 0] is also [output > 0]: relu keeps exactly the
    // positive entries. It is read from the output while that is unchanged,
    // so an input that is a deferred product never has to be computed; the
    // input's version is checked either way, as the reference's rule does.
    const detail::SavedTensor saved(v), saved_out(out);
    const auto mask = [saved, saved_out] {
        const Tensor input = saved.unpack();
        std::optional<Tensor> output = saved_out.unpack_if_unchanged();
        return output ? *output : input;
    };
    detail::attach_grad_fn(out, {v}, [mask](const Tensor& g) {
        return std::vector<Tensor>{activation_grad(HipBackend::Activation::Relu, g, mask())};
    });
    if (out.impl()->grad_fn) out.impl()->grad_fn->relu_mask = mask;
    return out;
}

Tensor sigmoid(const Tensor& v) {
    auto out = unary_forward(v, cpu::UnaryOp::Sigmoid);
    const detail::SavedTensor saved(out);
    detail::attach_grad_fn(out, {v}, [saved](const Tensor& g) {
        return std::vector<Tensor>{activation_grad(HipBackend::Activation::Sigmoid, g, saved.unpack())};
    });
    return out;
}

// log_softmax(x) = (x - m) - log(sum(exp(x - m))), m = max(x.detach()): the
// shift keeps exp() finite and, being constant, leaves the gradient exact.
Tensor log_softmax(const Tensor& v, std::int64_t axis) {
    const Tensor shifted = v - max(v.detach(), axis, true);
    return shifted - log(sum(exp(shifted), axis, true));
}

Tensor softmax(const Tensor& v, std::int64_t axis) { return exp(log_softmax(v, axis)); }

}  // namespace vectorcore
