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

#include <algorithm>
#include <atomic>
#include <cstdlib>
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

// The state of every hip storage (buffer, host shadow, deferred product,
// readers) is guarded by one recursive mutex: computing a deferred product
// reads its operands, which may be deferred products themselves.
std::recursive_mutex& state_mutex() {
    static std::recursive_mutex mu;
    return mu;
}

class HipStorage;

// A forward product recorded but not launched yet:
// C = A [m, k] @ B [k, n] (+ bias [n] on every row) (then ReLU), all contiguous.
struct DeferredProduct {
    std::shared_ptr<HipStorage> a, b, bias;
    std::size_t a_offset = 0, b_offset = 0, bias_offset = 0;
    std::size_t m = 0, k = 0, n = 0;
    bool relu = false;

    [[nodiscard]] bool reads(const HipStorage* s) const { return a.get() == s || b.get() == s || bias.get() == s; }
    void replace(const HipStorage* s, const std::shared_ptr<HipStorage>& with) {
        if (a.get() == s) a = with;
        if (b.get() == s) b = with;
        if (bias.get() == s) bias = with;
    }
};

class HipStorage final : public Storage, public std::enable_shared_from_this<HipStorage> {
public:
    // A fresh pooled buffer of `elements` floats (contents undefined).
    explicit HipStorage(std::size_t elements) : elements_(elements), shadow_valid_(false) {
        check(vc_hip_alloc(bytes(), &ptr_), "HIP allocation failed");
    }
    // A small tensor from host values: kept on the host until a kernel needs it.
    HipStorage(const float* values, std::size_t elements)
        : elements_(elements), shadow_(values, values + elements), shadow_valid_(true) {}
    // A product computed on first use (see ptr()).
    HipStorage(std::size_t elements, DeferredProduct product)
        : elements_(elements), deferred_(std::make_unique<DeferredProduct>(std::move(product))), shadow_valid_(false) {}
    // Takes over a pooled buffer that already holds this storage's contents.
    HipStorage(std::size_t elements, void* buffer) : elements_(elements), ptr_(buffer), shadow_valid_(false) {}

    ~HipStorage() override {
        if (mirror_) (void)vc_hip_mirror_release(mirror_);
        if (ptr_) (void)vc_hip_release(ptr_);
    }
    HipStorage(const HipStorage&) = delete;
    HipStorage& operator=(const HipStorage&) = delete;

    [[nodiscard]] Device device() const noexcept override { return Device::hip(); }
    [[nodiscard]] std::size_t size() const noexcept override { return elements_; }

    // The device buffer, allocated, uploaded or computed (a deferred product)
    // on first use.
    float* ptr() const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        if (!ptr_) {
            check(vc_hip_alloc(bytes(), &ptr_), "HIP allocation failed");
            if (!shadow_.empty()) check(vc_hip_upload(ptr_, shadow_.data(), shadow_.size() * sizeof(float)), "HIP upload failed");
        }
        if (deferred_) {
            const DeferredProduct& d = *deferred_;
            check(vc_hip_matmul_bias_relu(d.a->ptr() + d.a_offset, d.b->ptr() + d.b_offset, static_cast<float*>(ptr_),
                                          d.m, d.k, d.n, d.bias ? d.bias->ptr() + d.bias_offset : nullptr,
                                          d.relu ? 1 : 0),
                  "HIP matmul failed");
            deferred_.reset();  // drops the operands
        }
        return static_cast<float*>(ptr_);
    }

    std::optional<float> host_scalar() const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        if (elements_ == 1 && shadow_valid_ && shadow_.size() == 1) return shadow_[0];
        return std::nullopt;
    }

    // Host copy readable without a full synchronisation: the host shadow, or
    // the published value of a one-element result (waits for its producer only).
    bool host_copy(std::size_t offset, float* dst, std::size_t n) const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        if (mirror_ && elements_ == 1 && offset == 0 && n == 1) {
            check(vc_hip_mirror_read(mirror_, dst), "HIP command failed");
            return true;
        }
        if (!shadow_valid_ || shadow_.empty()) return false;
        std::copy(shadow_.begin() + static_cast<std::ptrdiff_t>(offset),
                  shadow_.begin() + static_cast<std::ptrdiff_t>(offset + n), dst);
        return true;
    }

    // Publishes this one-element storage's value, as computed so far in stream
    // order, for host_copy (vc_hip_mirror_scalar).
    void publish() {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        if (elements_ != 1) return;
        vc_hip_mirror* m = nullptr;
        check(vc_hip_mirror_scalar(ptr(), &m), "HIP launch failed");
        if (mirror_) (void)vc_hip_mirror_release(mirror_);
        mirror_ = m;
    }

    // Column sums of this storage's contents as [rows, cols], computed by the
    // kernel that wrote it (a bias gradient). Kept until taken or until the
    // storage is written in place.
    void set_column_sum(std::shared_ptr<HipStorage> sums, std::size_t rows, std::size_t cols) {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        column_sum_ = std::move(sums);
        column_sum_rows_ = rows;
        column_sum_cols_ = cols;
    }
    // The column sums for a [rows, cols] view of the whole storage, once.
    std::shared_ptr<HipStorage> take_column_sum(std::size_t rows, std::size_t cols) const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        if (!column_sum_ || rows != column_sum_rows_ || cols != column_sum_cols_ || rows * cols != elements_)
            return nullptr;
        return std::move(column_sum_);
    }

    // The deferred product this storage still has to compute, if any (a copy
    // for building a product with a longer epilogue).
    std::optional<DeferredProduct> pending() const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        if (!deferred_) return std::nullopt;
        return *deferred_;
    }

    // Records `reader` as a deferred product that reads this storage.
    void add_reader(const std::shared_ptr<HipStorage>& reader) {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        readers_.erase(std::remove_if(readers_.begin(), readers_.end(), [](const auto& w) { return w.expired(); }),
                       readers_.end());
        readers_.push_back(reader);
    }

    // Before an in-place write of elements [offset, offset + count) of this
    // storage. Deferred products that read it and have not run yet must still
    // see the current contents: the current buffer moves to a new read-only
    // storage that those products read from, and this storage continues with
    // a fresh buffer (holding a copy of the old contents unless the write
    // covers all of it). Returns the storage whose buffer holds the current
    // contents (this one when nothing was deferred on it); the caller keeps it
    // alive until the write is enqueued and writes its result into ptr().
    std::shared_ptr<const HipStorage> before_write(std::size_t offset, std::size_t count) {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        (void)ptr();
        shadow_valid_ = false;
        column_sum_.reset();  // about to be stale
        if (mirror_) {  // the published value is about to be stale
            (void)vc_hip_mirror_release(mirror_);
            mirror_ = nullptr;
        }
        std::vector<std::shared_ptr<HipStorage>> waiting;
        for (const auto& w : readers_) {
            auto r = w.lock();
            if (r && r->deferred_ && r->deferred_->reads(this)) waiting.push_back(std::move(r));
        }
        if (waiting.empty()) {
            readers_.clear();
            return shared_from_this();
        }
        void* fresh_buffer = nullptr;
        check(vc_hip_alloc(bytes(), &fresh_buffer), "HIP allocation failed");
        if (offset != 0 || count != elements_) {
            const int status = vc_hip_copy(fresh_buffer, ptr_, bytes());
            if (status != VC_HIP_OK) {
                (void)vc_hip_release(fresh_buffer);
                throw_status(status, "HIP copy failed");
            }
        }
        auto previous = std::make_shared<HipStorage>(elements_, ptr_);  // takes over the current buffer
        ptr_ = fresh_buffer;
        for (const auto& r : waiting) {
            r->deferred_->replace(this, previous);
            previous->readers_.push_back(r);
        }
        readers_.clear();
        return previous;
    }

private:
    std::size_t bytes() const { return (elements_ ? elements_ : 1) * sizeof(float); }

    std::size_t elements_;
    mutable void* ptr_ = nullptr;
    std::vector<float> shadow_;
    mutable std::unique_ptr<DeferredProduct> deferred_;
    std::vector<std::weak_ptr<HipStorage>> readers_;
    vc_hip_mirror* mirror_ = nullptr;  // published value of a one-element result
    mutable std::shared_ptr<HipStorage> column_sum_;  // see set_column_sum
    std::size_t column_sum_rows_ = 0, column_sum_cols_ = 0;
    bool shadow_valid_;
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
void HipBackend::set_gemm_kernel(const std::string& name) {
    require(*this);
    check(vc_hip_set_gemm_kernel(name.c_str()), "HIP GEMM kernel selection failed");
}

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
                                                      bool trans_b, const Storage& mask,
                                                      std::size_t mask_offset, bool column_sum) {
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
    if (column_sum && batch == 1 && a_offsets[0] == 0 && b_offsets[0] == 0) {
        auto sums = fresh(n);
        check(vc_hip_matmul_relu_mask_colsum(dptr(a, a_offset), dptr(b, b_offset), out->ptr(), m, k, n, trans_a ? 1 : 0,
                                             trans_b ? 1 : 0, dptr(mask, mask_offset), sums->ptr()),
              "HIP matmul failed");
        out->set_column_sum(std::move(sums), m, n);
        return out;
    }
    check(vc_hip_matmul_relu_mask(dptr(a, a_offset), dptr(b, b_offset), out->ptr(), m, k, n, a_offsets.data(),
                                  b_offsets.data(), batch, trans_a ? 1 : 0, trans_b ? 1 : 0,
                                  dptr(mask, mask_offset)),
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
    out->publish();  // item() on the sum then waits for this point of the stream only
    return out;
}

std::shared_ptr<Storage> HipBackend::reduce_axis(const Storage& input, std::size_t offset, std::size_t outer,
                                                 std::size_t length, std::size_t inner, cpu::ReduceOp operation) {
    require(*this);
    if (length == 0 && operation != cpu::ReduceOp::Sum)
        throw std::invalid_argument("max/argmax over an empty axis is undefined");
    if (operation == cpu::ReduceOp::Sum && outer == 1 && offset == 0) {
        // Column sums the kernel that wrote the input already produced.
        if (auto sums = as_hip(input).take_column_sum(length, inner)) return sums;
    }
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
    axpy_batch({AxpyItem{&target, target_offset, &source, source_offset, count}}, alpha);
}

void HipBackend::axpy_batch(const std::vector<AxpyItem>& items, float alpha) {
    require(*this);
    for (const AxpyItem& it : items) {
        if (it.target_offset + it.count > it.target->size() || it.source_offset + it.count > it.source->size())
            throw std::out_of_range("HIP axpy exceeds storage");
        (void)as_hip(*it.target);
    }
    std::vector<std::shared_ptr<const HipStorage>> current;  // kept alive until the launch is enqueued
    std::vector<float*> outputs;
    std::vector<const float*> targets, sources;
    std::vector<std::size_t> counts;
    for (const AxpyItem& it : items) {
        auto& t = as_hip(*it.target);
        current.push_back(t.before_write(it.target_offset, it.count));
        if (it.count == 0) continue;
        outputs.push_back(t.ptr() + it.target_offset);
        targets.push_back(current.back()->ptr() + it.target_offset);
        // A source in the target's own storage (a gradient that aliases its
        // parameter, e.g. from w.backward(w)) is read from the buffer holding
        // the current contents: before_write may have given the target a
        // fresh, unwritten buffer.
        sources.push_back(it.source == it.target ? current.back()->ptr() + it.source_offset
                                                 : dptr(*it.source, it.source_offset));
        counts.push_back(it.count);
    }
    if (outputs.empty()) return;
    check(vc_hip_axpy_batch(outputs.data(), targets.data(), sources.data(), counts.data(), outputs.size(), alpha),
          "HIP axpy failed");
}

namespace {
std::atomic<bool>& defer_flag() {
    static std::atomic<bool> flag{[] {
        const char* v = std::getenv("VECTORCORE_HIP_DEFER");
        return !(v && std::string(v) == "0");
    }()};
    return flag;
}
}  // namespace

void HipBackend::set_defer_products(bool enable) { defer_flag() = enable; }
bool HipBackend::defer_products() const { return defer_flag(); }

std::shared_ptr<Storage> HipBackend::matmul_deferred(const std::shared_ptr<Storage>& a, std::size_t a_offset,
                                                     const std::shared_ptr<Storage>& b, std::size_t b_offset,
                                                     std::size_t m, std::size_t k, std::size_t n) {
    require(*this);
    if (!defer_products() || m == 0 || k == 0 || n == 0) return nullptr;
    auto ha = std::dynamic_pointer_cast<HipStorage>(a), hb = std::dynamic_pointer_cast<HipStorage>(b);
    if (!ha || !hb) throw std::invalid_argument("expected HIP storage");
    if (a_offset + m * k > ha->size() || b_offset + k * n > hb->size())
        throw std::out_of_range("HIP matmul operand exceeds storage");
    // An operand that is itself a deferred product is computed now: nothing
    // more can join its epilogue once a product reads it, launching it here
    // lets the device start while the host records the rest, and no record
    // ever waits on another (computing one never recurses).
    (void)ha->ptr();
    (void)hb->ptr();
    DeferredProduct d;
    d.a = ha;
    d.b = hb;
    d.a_offset = a_offset;
    d.b_offset = b_offset;
    d.m = m;
    d.k = k;
    d.n = n;
    auto out = std::make_shared<HipStorage>(m * n, std::move(d));
    ha->add_reader(out);
    hb->add_reader(out);
    return out;
}

std::shared_ptr<Storage> HipBackend::add_bias_deferred(const Storage& product, std::size_t product_offset,
                                                       const Shape& product_shape, const Strides& product_strides,
                                                       const std::shared_ptr<Storage>& bias, std::size_t bias_offset,
                                                       const Shape& bias_shape, const Strides& bias_strides) {
    const auto* hp = dynamic_cast<const HipStorage*>(&product);
    auto hbias = std::dynamic_pointer_cast<HipStorage>(bias);
    if (!hp || !hbias || product_offset != 0 || product_shape.size() != 2) return nullptr;
    std::optional<DeferredProduct> d = hp->pending();
    if (!d || d->bias || d->relu || product_shape[0] != d->m || product_shape[1] != d->n ||
        product_strides != contiguous_strides(product_shape))
        return nullptr;
    const bool row = (bias_shape == Shape{d->n} || bias_shape == Shape{1, d->n}) &&
                     bias_strides == contiguous_strides(bias_shape) && bias_offset + d->n <= hbias->size();
    if (!row) return nullptr;
    (void)hbias->ptr();  // a deferred bias is computed now, as a product's operands are
    d->bias = hbias;
    d->bias_offset = bias_offset;
    auto out = std::make_shared<HipStorage>(d->m * d->n, *d);
    d->a->add_reader(out);
    d->b->add_reader(out);
    hbias->add_reader(out);
    return out;
}

std::shared_ptr<Storage> HipBackend::relu_deferred(const Storage& input, std::size_t offset, std::size_t count) {
    const auto* h = dynamic_cast<const HipStorage*>(&input);
    if (!h || offset != 0) return nullptr;
    std::optional<DeferredProduct> d = h->pending();
    if (!d || d->relu || count != d->m * d->n) return nullptr;
    d->relu = true;
    auto out = std::make_shared<HipStorage>(count, *d);
    d->a->add_reader(out);
    d->b->add_reader(out);
    if (d->bias) d->bias->add_reader(out);
    return out;
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
    loss->publish();  // loss.item() then waits for the forward only, not the backward and update after it
    return {loss, stats};
}

std::shared_ptr<Storage> HipBackend::cross_entropy_backward(const Storage& logits, std::size_t logits_offset,
                                                            const Storage& targets, const Storage& row_stats,
                                                            const Storage& grad_loss, std::size_t grad_offset,
                                                            std::size_t rows, std::size_t classes, bool column_sum) {
    require(*this);
    auto out = fresh(rows * classes);
    const auto* t = reinterpret_cast<const std::int32_t*>(as_hip(targets).ptr());
    // backward()'s seed is a host-known scalar: pass its value, no upload.
    const std::optional<float> seed = grad_offset == 0 ? hip_host_scalar(grad_loss) : std::nullopt;
    if (column_sum && classes > 0) {
        auto sums = fresh(classes);
        check(vc_hip_xent_backward_colsum(dptr(logits, logits_offset), t, as_hip(row_stats).ptr(),
                                          seed ? nullptr : dptr(grad_loss, grad_offset), seed ? *seed : 0.0F, rows,
                                          classes, out->ptr(), sums->ptr()),
              "HIP cross-entropy backward failed");
        out->set_column_sum(std::move(sums), rows, classes);
        return out;
    }
    const int status =
        seed ? vc_hip_xent_backward_value(dptr(logits, logits_offset), t, as_hip(row_stats).ptr(), *seed, rows, classes,
                                          out->ptr())
             : vc_hip_xent_backward(dptr(logits, logits_offset), t, as_hip(row_stats).ptr(),
                                    dptr(grad_loss, grad_offset), rows, classes, out->ptr());
    check(status, "HIP cross-entropy backward failed");
    return out;
}

std::optional<float> hip_host_scalar(const Storage& storage) {
    const auto* h = dynamic_cast<const HipStorage*>(&storage);
    return h ? h->host_scalar() : std::nullopt;
}

bool hip_available() { return HipBackend::instance().available(); }
std::string hip_device_name() { return HipBackend::instance().device_name(); }

}  // namespace vectorcore
