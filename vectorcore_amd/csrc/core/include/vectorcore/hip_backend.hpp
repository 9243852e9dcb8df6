#pragma once
// The `hip` device: a C++ wrapper over the C ABI of include/vc_hip.h.
//
// HipBackend keeps the member set of the reference's device interface
// (MetalBackend, include/vectorcore/metal_backend.hpp:13-56) so the dispatch
// sites of ops/tensor/autograd/nn call it the same way, and adds the fused
// backward kernels that the hip arm of those sites uses. Every member throws
// the reference's exception types; there is no CPU fallback.
#include "vectorcore/cpu_backend.hpp"
#include "vectorcore/shape.hpp"
#include "vectorcore/storage.hpp"

#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <utility>
#include <vector>

namespace vectorcore {

class HipBackend {
public:
    static HipBackend& instance();

    [[nodiscard]] bool available() const noexcept;
    [[nodiscard]] std::string device_name() const;
    [[nodiscard]] std::string last_error() const;
    // "mfma" (matrix-core tiles), "simple" (VECTORCORE_HIP_GEMM=simple) or "unavailable".
    [[nodiscard]] std::string gemm_kernel() const;
    // "mfma", "simple", "mfma128" or "mfma256" for later products (vc_hip_set_gemm_kernel).
    void set_gemm_kernel(const std::string& name);

    // --- the reference device interface ---
    [[nodiscard]] std::shared_ptr<Storage> allocate(std::size_t elements);
    [[nodiscard]] std::shared_ptr<Storage> upload(const float* data, std::size_t elements);
    void download(const Storage& source, std::size_t offset, float* destination, std::size_t elements);
    [[nodiscard]] std::shared_ptr<Storage> binary(const Storage& a, std::size_t a_offset, const Shape& a_shape,
                                                  const Strides& a_strides, const Storage& b, std::size_t b_offset,
                                                  const Shape& b_shape, const Strides& b_strides,
                                                  const Shape& out_shape, cpu::BinaryOp operation);
    [[nodiscard]] std::shared_ptr<Storage> unary(const Storage& input, std::size_t offset, std::size_t count,
                                                 cpu::UnaryOp operation);
    // Output z is op(A + a_offsets[z]) @ op(B + b_offsets[z]) (offsets in elements).
    [[nodiscard]] std::shared_ptr<Storage> matmul(const Storage& a, std::size_t a_offset, const Storage& b,
                                                  std::size_t b_offset, std::size_t m, std::size_t k, std::size_t n,
                                                  const std::vector<std::size_t>& a_offsets,
                                                  const std::vector<std::size_t>& b_offsets, bool trans_a,
                                                  bool trans_b);
    // matmul() followed by the ReLU backward rule in the same kernel: the output
    // is multiplied by [mask > 0] (mask: the ReLU's input or output, laid out
    // like the product). column_sum (one product only): the kernel also
    // produces the output's column sums, which stay with the output storage
    // until reduce_axis asks for exactly that sum (or the storage is written).
    [[nodiscard]] std::shared_ptr<Storage> matmul_relu_mask(const Storage& a, std::size_t a_offset, const Storage& b,
                                                            std::size_t b_offset, std::size_t m, std::size_t k,
                                                            std::size_t n, const std::vector<std::size_t>& a_offsets,
                                                            const std::vector<std::size_t>& b_offsets, bool trans_a,
                                                            bool trans_b, const Storage& mask,
                                                            std::size_t mask_offset, bool column_sum = false);
    [[nodiscard]] std::shared_ptr<Storage> transpose_last2(const Storage& input, std::size_t offset, std::size_t batch,
                                                           std::size_t rows, std::size_t cols);
    [[nodiscard]] std::shared_ptr<Storage> reduce_sum(const Storage& input, std::size_t offset, std::size_t count);
    [[nodiscard]] std::shared_ptr<Storage> reduce_axis(const Storage& input, std::size_t offset, std::size_t outer,
                                                       std::size_t length, std::size_t inner, cpu::ReduceOp operation);
    [[nodiscard]] std::shared_ptr<Storage> scatter_axis(const Storage& values, std::size_t values_offset,
                                                        const Storage& indices, std::size_t indices_offset,
                                                        std::size_t outer, std::size_t length, std::size_t inner);
    void axpy_inplace(Storage& target, std::size_t target_offset, const Storage& source, std::size_t source_offset,
                      std::size_t count, float alpha);
    // axpy_inplace for several (target, source) pairs in one pass. A target
    // must not overlap another pair's target or source; the result is then the
    // same bits as one axpy_inplace per pair.
    struct AxpyItem {
        Storage* target;
        std::size_t target_offset;
        const Storage* source;
        std::size_t source_offset;
        std::size_t count;
    };
    void axpy_batch(const std::vector<AxpyItem>& items, float alpha);
    void synchronize();
    // download() of a published one-element result (a loss or a full sum)
    // normally waits for its producer only, so item() can return while later
    // work still runs. Strict mode restores the reference's contract
    // (metal_backend.mm:198-211): every download first waits for the whole
    // stream and reports any asynchronous failure. Off by default;
    // VECTORCORE_HIP_STRICT_ITEM=1 or set_strict_item(true) turns it on.
    void set_strict_item(bool enable);
    [[nodiscard]] bool strict_item() const;

    // --- deferred forward products ---
    // A 2-D product A [m, k] @ B [k, n] (contiguous) can be recorded instead of
    // launched; it is computed the first time its storage is read. Until then
    // a row-bias add and a ReLU applied to it become a new deferred product
    // with that epilogue, computed by one kernel (vc_hip_matmul_bias_relu),
    // and the partial results nobody reads are never computed. An in-place
    // write to an operand of a product still deferred first moves the
    // operand's current buffer to that product (axpy_batch), so results are
    // those of eager execution. Each returns null when it does not apply; the
    // caller then runs the op eagerly.
    [[nodiscard]] std::shared_ptr<Storage> matmul_deferred(const std::shared_ptr<Storage>& a, std::size_t a_offset,
                                                           const std::shared_ptr<Storage>& b, std::size_t b_offset,
                                                           std::size_t m, std::size_t k, std::size_t n);
    // product + bias, product a whole deferred product [m, n] without epilogue
    // and bias a contiguous [n] or [1, n].
    [[nodiscard]] std::shared_ptr<Storage> add_bias_deferred(const Storage& product, std::size_t product_offset,
                                                             const Shape& product_shape, const Strides& product_strides,
                                                             const std::shared_ptr<Storage>& bias,
                                                             std::size_t bias_offset, const Shape& bias_shape,
                                                             const Strides& bias_strides);
    // relu(input), input a whole deferred product without ReLU.
    [[nodiscard]] std::shared_ptr<Storage> relu_deferred(const Storage& input, std::size_t offset, std::size_t count);
    // On by default; VECTORCORE_HIP_DEFER=0 or set_defer_products(false) makes
    // every product eager.
    void set_defer_products(bool enable);
    [[nodiscard]] bool defer_products() const;

    // --- deferred elementwise expressions ---
    // While an ElementwiseScope is alive on this thread (the autograd engine
    // opens one for a backward pass), binary, binary_scalar, negate and
    // ReLU-gradient unary ops, activation_backward and divide_backward on
    // same-shape contiguous operands, and column sums of their results
    // (reduce_axis, outer 1), record an expression instead of launching a
    // kernel. A storage holding one is computed by one vc_hip_map program on
    // first use; flush_elementwise computes every such storage of the scope
    // still referenced, those over the same elements in one program, and the
    // intermediate values nothing references any more are never written.
    // Elementwise values are the same bits as the eager kernels'. Column sums
    // are added in a different fixed order from reduce_axis's: deterministic
    // for either setting, they can differ in the last bit between the two. On
    // by default; VECTORCORE_HIP_FUSE=0 or set_fuse_elementwise(false) keeps
    // every op eager.
    class ElementwiseScope {
    public:
        ElementwiseScope();
        ~ElementwiseScope();
        ElementwiseScope(const ElementwiseScope&) = delete;
        ElementwiseScope& operator=(const ElementwiseScope&) = delete;
    };
    void flush_elementwise();
    void set_fuse_elementwise(bool enable);
    [[nodiscard]] bool fuse_elementwise() const;

    // --- fused kernels used by the hip arm of the backward rules ---
    [[nodiscard]] std::shared_ptr<Storage> fill(std::size_t count, float value);
    // out = a op s (scalar_first false) or s op a; s is a host value.
    [[nodiscard]] std::shared_ptr<Storage> binary_scalar(const Storage& a, std::size_t a_offset, std::size_t count,
                                                         float s, bool scalar_first, cpu::BinaryOp operation);
    // The broadcast-batch gradient: sum_z op(A + z*a_stride) @ op(B + z*b_stride).
    [[nodiscard]] std::shared_ptr<Storage> matmul_reduce(const Storage& a, std::size_t a_offset, const Storage& b,
                                                         std::size_t b_offset, std::size_t m, std::size_t k,
                                                         std::size_t n, std::size_t count, std::size_t a_stride,
                                                         std::size_t b_stride, bool trans_a, bool trans_b);
    enum class Activation { Relu, Sigmoid, Exp, Log };
    // relu: grad * [input > 0]; sigmoid: (grad * y) * (1 - y); exp: grad * y; log: grad / input.
    [[nodiscard]] std::shared_ptr<Storage> activation_backward(Activation kind, const Storage& grad,
                                                               std::size_t grad_offset, const Storage& saved,
                                                               std::size_t saved_offset, std::size_t count);
    // Division gradients over out_shape: {grad / b, -(grad * a) / (b * b)} (either may be skipped).
    std::pair<std::shared_ptr<Storage>, std::shared_ptr<Storage>> divide_backward(
        const Storage& grad, std::size_t grad_offset, const Storage& a, std::size_t a_offset, const Shape& a_shape,
        const Strides& a_strides, const Storage& b, std::size_t b_offset, const Shape& b_shape,
        const Strides& b_strides, const Shape& out_shape, bool need_a, bool need_b);
    // Class indices as int32 on the device (caller has range-checked them).
    [[nodiscard]] std::shared_ptr<Storage> upload_targets(const std::vector<std::size_t>& targets);
    // Returns {loss (1 element), row statistics (2 per row)}.
    std::pair<std::shared_ptr<Storage>, std::shared_ptr<Storage>> cross_entropy_forward(
        const Storage& logits, std::size_t logits_offset, const Storage& targets, std::size_t rows,
        std::size_t classes);
    // column_sum: the kernel also produces the gradient's column sums, kept
    // with the returned storage for reduce_axis (as matmul_relu_mask does).
    [[nodiscard]] std::shared_ptr<Storage> cross_entropy_backward(const Storage& logits, std::size_t logits_offset,
                                                                  const Storage& targets, const Storage& row_stats,
                                                                  const Storage& grad_loss, std::size_t grad_offset,
                                                                  std::size_t rows, std::size_t classes,
                                                                  bool column_sum = false);
};

// Host-side value of a one-element hip storage created from host data, if it
// has not been written on the device since (lets scalar operands skip a
// device read).
std::optional<float> hip_host_scalar(const Storage& storage);

[[nodiscard]] bool hip_available();
[[nodiscard]] std::string hip_device_name();

}  // namespace vectorcore
