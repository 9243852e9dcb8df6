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
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>

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
// Layer products below this many outputs take kernels that write no ReLU
// bits (the 256-row tiles need a full round of workgroups): no bits buffer
// is requested for them.
constexpr std::size_t kReluBitsMinElements = std::size_t(1) << 20;

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

// One value of a deferred elementwise expression: an input buffer (a whole
// or offset view of a computed storage, `count` elements like the
// expression), a constant, or one fp32 operation (VC_MAP_*) on two values
// (b == a for the one-operand operations). Nodes are shared between the
// expressions built on them.
struct MapNode {
    enum class Kind { Input, Constant, Op };
    Kind kind = Kind::Op;
    int op = 0;
    std::shared_ptr<MapNode> a, b;
    std::shared_ptr<HipStorage> input;
    std::size_t offset = 0;
    float value = 0.0F;
};
using MapExpr = std::shared_ptr<MapNode>;

bool expr_reads(const MapNode& n, const HipStorage* s);
void expr_replace(MapNode& n, const HipStorage* s, const std::shared_ptr<HipStorage>& with);
void run_maps(const std::vector<HipStorage*>& outputs);

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
    // The values of a deferred elementwise expression (computed on first use
    // or by HipBackend::flush_elementwise).
    HipStorage(std::size_t elements, MapExpr expr) : elements_(elements), map_(std::move(expr)), shadow_valid_(false) {}
    // The column sums of a deferred expression viewed as [rows, elements].
    HipStorage(std::size_t elements, MapExpr expr, std::size_t rows)
        : elements_(elements), sum_of_(std::move(expr)), sum_rows_(rows), shadow_valid_(false) {}

    ~HipStorage() override {
        if (mirror_) (void)vc_hip_mirror_release(mirror_);
        if (pending_sums_) (void)vc_hip_colsum_release(pending_sums_);
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
        if (map_ || sum_of_) {
            run_maps({const_cast<HipStorage*>(this)});
            return static_cast<float*>(ptr_);
        }
        if (!ptr_) {
            check(vc_hip_alloc(bytes(), &ptr_), "HIP allocation failed");
            if (!shadow_.empty()) check(vc_hip_upload(ptr_, shadow_.data(), shadow_.size() * sizeof(float)), "HIP upload failed");
        }
        if (pending_sums_) {
            check(vc_hip_colsum_finish(pending_sums_, static_cast<float*>(ptr_)), "HIP column sum failed");
            (void)vc_hip_colsum_release(pending_sums_);
            pending_sums_ = nullptr;
        }
        if (deferred_) {
            const DeferredProduct& d = *deferred_;
            const float* bias = d.bias ? d.bias->ptr() + d.bias_offset : nullptr;
            if (d.relu && d.m * d.n >= kReluBitsMinElements) {
                // With the layer's ReLU bitmask where its kernel writes one,
                // for the product that applies the ReLU's backward rule.
                auto bits = std::make_shared<HipStorage>((d.m + 31) / 32 * d.n);
                int written = 0;
                check(vc_hip_matmul_bias_relu_bits(d.a->ptr() + d.a_offset, d.b->ptr() + d.b_offset,
                                                   static_cast<float*>(ptr_), d.m, d.k, d.n, bias,
                                                   reinterpret_cast<uint32_t*>(bits->ptr()), &written),
                      "HIP matmul failed");
                if (written) {
                    relu_bits_ = std::move(bits);
                    relu_bits_rows_ = d.m;
                    relu_bits_cols_ = d.n;
                }
            } else {
                check(vc_hip_matmul_bias_relu(d.a->ptr() + d.a_offset, d.b->ptr() + d.b_offset,
                                              static_cast<float*>(ptr_), d.m, d.k, d.n, bias, d.relu ? 1 : 0),
                      "HIP matmul failed");
            }
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
        adopt_mirror(m);
    }

    // Takes a mirror already published from this one-element storage (its
    // producer wrote the host slot, vc_hip_xent_forward_published).
    void adopt_mirror(vc_hip_mirror* m) {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
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

    // This storage's values are the column sums that `sums` leaves pending
    // (the partial rows of the kernel that wrote the summed matrix); they are
    // finished into the buffer on first read, and an optimizer step can take
    // them unfinished (pending_sums).
    void set_pending_sums(vc_hip_colsum* sums) {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        if (pending_sums_) (void)vc_hip_colsum_release(pending_sums_);
        pending_sums_ = sums;
    }
    const vc_hip_colsum* pending_sums() const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        return pending_sums_;
    }

    // Argmax along the last axis of this storage's [rows, cols] view at
    // `offset`, computed by a kernel that read those rows (the cross-entropy
    // forward). Kept until taken or until the storage is written in place.
    void set_row_argmax(std::shared_ptr<HipStorage> indices, std::size_t offset, std::size_t rows,
                        std::size_t cols) const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        row_argmax_ = std::move(indices);
        row_argmax_offset_ = offset;
        row_argmax_rows_ = rows;
        row_argmax_cols_ = cols;
    }
    // The argmax kept for exactly that view, once.
    std::shared_ptr<HipStorage> take_row_argmax(std::size_t offset, std::size_t rows, std::size_t cols) const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        if (!row_argmax_ || offset != row_argmax_offset_ || rows != row_argmax_rows_ || cols != row_argmax_cols_)
            return nullptr;
        return std::move(row_argmax_);
    }

    // The ReLU bitmask ([value > 0], in vc_hip_matmul_bias_relu_bits' layout)
    // of this storage's contents as [rows, cols], written by the fused layer
    // product that computed them. Kept until the storage is written in place.
    const uint32_t* relu_bits(std::size_t rows, std::size_t cols) const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        if (!relu_bits_ || rows != relu_bits_rows_ || cols != relu_bits_cols_ || rows * cols != elements_)
            return nullptr;
        return reinterpret_cast<const uint32_t*>(relu_bits_->ptr());
    }

    // The deferred product this storage still has to compute, if any (a copy
    // for building a product with a longer epilogue).
    std::optional<DeferredProduct> pending() const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        if (!deferred_) return std::nullopt;
        return *deferred_;
    }

    // The pending elementwise expression of this storage, if any.
    MapExpr map_expr() const {
        std::lock_guard<std::recursive_mutex> lock(state_mutex());
        return map_;
    }
    MapExpr sum_expr() const { return sum_of_; }
    std::size_t sum_rows() const { return sum_rows_; }
    bool map_pending() const { return map_ != nullptr || sum_of_ != nullptr; }
    // Takes the buffer a program wrote this storage's values into, and drops
    // the expression (and with it the references to its inputs).
    void set_computed(void* buffer) {
        ptr_ = buffer;
        map_.reset();
        sum_of_.reset();
    }

    // Records `reader` as a deferred product or expression that reads this storage.
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
        row_argmax_.reset();
        relu_bits_.reset();
        if (mirror_) {  // the published value is about to be stale
            (void)vc_hip_mirror_release(mirror_);
            mirror_ = nullptr;
        }
        std::vector<std::shared_ptr<HipStorage>> waiting;
        for (const auto& w : readers_) {
            auto r = w.lock();
            if (r && r.get() != this && r->reads_pending(this)) waiting.push_back(std::move(r));
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
            if (r->deferred_) r->deferred_->replace(this, previous);
            if (r->map_) expr_replace(*r->map_, this, previous);
            if (r->sum_of_) expr_replace(*r->sum_of_, this, previous);
            previous->readers_.push_back(r);
        }
        readers_.clear();
        return previous;
    }

private:
    std::size_t bytes() const { return (elements_ ? elements_ : 1) * sizeof(float); }
    // Does work still deferred on this storage read s?
    bool reads_pending(const HipStorage* s) const {
        return (deferred_ && deferred_->reads(s)) || (map_ && expr_reads(*map_, s)) || (sum_of_ && expr_reads(*sum_of_, s));
    }

    std::size_t elements_;
    mutable void* ptr_ = nullptr;
    std::vector<float> shadow_;
    mutable std::unique_ptr<DeferredProduct> deferred_;
    mutable MapExpr map_;     // deferred elementwise values
    mutable MapExpr sum_of_;  // deferred column sums of this expression
    std::size_t sum_rows_ = 0;
    std::vector<std::weak_ptr<HipStorage>> readers_;
    vc_hip_mirror* mirror_ = nullptr;  // published value of a one-element result
    mutable vc_hip_colsum* pending_sums_ = nullptr;  // see set_pending_sums
    mutable std::shared_ptr<HipStorage> column_sum_;  // see set_column_sum
    std::size_t column_sum_rows_ = 0, column_sum_cols_ = 0;
    mutable std::shared_ptr<HipStorage> row_argmax_;  // see set_row_argmax
    mutable std::size_t row_argmax_offset_ = 0, row_argmax_rows_ = 0, row_argmax_cols_ = 0;
    mutable std::shared_ptr<HipStorage> relu_bits_;  // see relu_bits
    mutable std::size_t relu_bits_rows_ = 0, relu_bits_cols_ = 0;
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

// ---- deferred elementwise expressions ------------------------------------------
// During a backward pass (an ElementwiseScope on this thread), the elementwise
// rules on same-shape contiguous operands record expressions instead of
// launching one kernel per operation. An expression is computed by one
// vc_hip_map program when its storage is first read, or, together with every
// other expression of the pass that is still referenced, when the pass ends
// (flush_elementwise); intermediate results that only fed other expressions
// are never written. A column sum (the bias gradient, sum_to_shape) of an
// expression becomes one more output of the program.

void collect(const MapNode* n, std::unordered_map<const MapNode*, int>& seen, std::vector<const MapNode*>& order) {
    if (seen.count(n)) return;
    seen.emplace(n, 0);
    if (n->kind == MapNode::Kind::Op) {
        collect(n->a.get(), seen, order);
        collect(n->b.get(), seen, order);
    }
    order.push_back(n);
}

bool expr_reads(const MapNode& root, const HipStorage* s) {
    std::unordered_map<const MapNode*, int> seen;
    std::vector<const MapNode*> order;
    collect(&root, seen, order);
    for (const MapNode* n : order)
        if (n->kind == MapNode::Kind::Input && n->input.get() == s) return true;
    return false;
}

void expr_replace(MapNode& root, const HipStorage* s, const std::shared_ptr<HipStorage>& with) {
    std::unordered_map<const MapNode*, int> seen;
    std::vector<const MapNode*> order;
    collect(&root, seen, order);
    for (const MapNode* n : order)
        if (n->kind == MapNode::Kind::Input && n->input.get() == s) const_cast<MapNode*>(n)->input = with;
}

// A vc_hip_map program for a set of expressions (roots), with slots assigned
// by liveness: inputs in [0, n_in), constants next, every operation's result
// in the lowest slot free at that point (an input's slot is free after its
// last use). Fails when the expressions need more inputs, constants,
// instructions or slots than one program has.
struct MapPlan {
    std::vector<const MapNode*> inputs;  // one node per distinct (storage, offset)
    std::vector<float> constants;
    std::vector<std::uint32_t> code;
    std::unordered_map<const MapNode*, int> root_slot;
};

bool plan_program(const std::vector<const MapNode*>& roots, MapPlan& plan) {
    std::unordered_map<const MapNode*, int> seen;
    std::vector<const MapNode*> order;
    for (const MapNode* r : roots) collect(r, seen, order);
    std::vector<const MapNode*> ops;
    std::vector<std::pair<const HipStorage*, std::size_t>> input_keys;
    std::vector<std::uint32_t> const_bits;
    std::unordered_map<const MapNode*, int> vid;  // value id: input index, then constants, then op index
    for (const MapNode* n : order) {
        if (n->kind == MapNode::Kind::Input) {
            const std::pair<const HipStorage*, std::size_t> key{n->input.get(), n->offset};
            auto it = std::find(input_keys.begin(), input_keys.end(), key);
            if (it == input_keys.end()) {
                input_keys.push_back(key);
                plan.inputs.push_back(n);
                it = input_keys.end() - 1;
            }
            vid[n] = static_cast<int>(it - input_keys.begin());
        } else if (n->kind == MapNode::Kind::Constant) {
            std::uint32_t bits = 0;
            std::memcpy(&bits, &n->value, sizeof bits);
            auto it = std::find(const_bits.begin(), const_bits.end(), bits);
            if (it == const_bits.end()) {
                const_bits.push_back(bits);
                plan.constants.push_back(n->value);
                it = const_bits.end() - 1;
            }
            vid[n] = -1 - static_cast<int>(it - const_bits.begin());  // resolved below
        } else {
            ops.push_back(n);
        }
    }
    const int n_in = static_cast<int>(plan.inputs.size()), n_const = static_cast<int>(plan.constants.size());
    if (n_in < 1 || n_in > VC_HIP_MAP_INPUTS || n_const > VC_HIP_MAP_CONSTANTS || n_in + n_const > VC_HIP_MAP_SLOTS ||
        ops.size() > VC_HIP_MAP_CODE)
        return false;
    for (auto& [n, v] : vid)
        if (v < 0) v = n_in + (-1 - v);
    for (std::size_t k = 0; k < ops.size(); ++k) vid[ops[k]] = n_in + n_const + static_cast<int>(k);
    // Last instruction reading each value; roots are read at the end.
    const int values = n_in + n_const + static_cast<int>(ops.size());
    std::vector<int> last_use(static_cast<std::size_t>(values), -1);
    for (std::size_t k = 0; k < ops.size(); ++k) {
        last_use[static_cast<std::size_t>(vid[ops[k]->a.get()])] = static_cast<int>(k);
        last_use[static_cast<std::size_t>(vid[ops[k]->b.get()])] = static_cast<int>(k);
    }
    for (const MapNode* r : roots) last_use[static_cast<std::size_t>(vid[r])] = static_cast<int>(ops.size());
    std::vector<int> slot(static_cast<std::size_t>(values), -1);
    std::vector<bool> busy(VC_HIP_MAP_SLOTS, false);
    for (int v = 0; v < n_in + n_const; ++v) {
        slot[static_cast<std::size_t>(v)] = v;
        busy[static_cast<std::size_t>(v)] = true;
    }
    for (std::size_t k = 0; k < ops.size(); ++k) {
        const int va = vid[ops[k]->a.get()], vb = vid[ops[k]->b.get()];
        const int sa = slot[static_cast<std::size_t>(va)], sb = slot[static_cast<std::size_t>(vb)];
        for (const int v : {va, vb}) {  // operands read for the last time free their slots (not constants)
            const bool constant = v >= n_in && v < n_in + n_const;
            if (!constant && last_use[static_cast<std::size_t>(v)] == static_cast<int>(k))
                busy[static_cast<std::size_t>(slot[static_cast<std::size_t>(v)])] = false;
        }
        int d = -1;
        for (int t = 0; t < VC_HIP_MAP_SLOTS && d < 0; ++t)
            if (!busy[static_cast<std::size_t>(t)] && !(t >= n_in && t < n_in + n_const)) d = t;
        if (d < 0) return false;
        busy[static_cast<std::size_t>(d)] = true;
        slot[static_cast<std::size_t>(n_in + n_const + static_cast<int>(k))] = d;
        plan.code.push_back(static_cast<std::uint32_t>(ops[k]->op) | static_cast<std::uint32_t>(sa) << 8 |
                            static_cast<std::uint32_t>(sb) << 16 | static_cast<std::uint32_t>(d) << 24);
    }
    for (const MapNode* r : roots) plan.root_slot[r] = slot[static_cast<std::size_t>(vid[r])];
    return true;
}

bool fits(const std::vector<const MapNode*>& roots) {
    MapPlan plan;
    return plan_program(roots, plan);
}

// Computes pending storages with one program: expressions (map outputs) and
// column sums, all over the same number of elements (and, for sums, the same
// columns). The caller holds the state mutex.
void run_maps(const std::vector<HipStorage*>& requested) {
    std::vector<HipStorage*> outputs;
    for (HipStorage* o : requested)
        if (o->map_pending()) outputs.push_back(o);
    std::vector<const MapNode*> roots;
    std::size_t count = 0, rows = 0, cols = 0;
    std::size_t n_out = 0, n_sum = 0;
    for (HipStorage* o : outputs) {
        if (MapExpr m = o->map_expr()) {
            roots.push_back(m.get());
            count = o->size();
            ++n_out;
        } else if (MapExpr e = o->sum_expr()) {
            roots.push_back(e.get());
            rows = o->sum_rows();
            cols = o->size();
            count = rows * cols;
            ++n_sum;
        }
    }
    if (roots.empty()) return;
    MapPlan plan;
    if (n_out > VC_HIP_MAP_OUTPUTS || n_sum > VC_HIP_MAP_SUMS || !plan_program(roots, plan))
        throw std::logic_error("deferred elementwise expression exceeds one program");
    vc_hip_map_program prog{};
    for (std::size_t j = 0; j < plan.inputs.size(); ++j)
        prog.inputs[j] = plan.inputs[j]->input->ptr() + plan.inputs[j]->offset;
    prog.n_inputs = plan.inputs.size();
    for (std::size_t c = 0; c < plan.constants.size(); ++c) prog.constants[c] = plan.constants[c];
    prog.n_constants = plan.constants.size();
    for (std::size_t k = 0; k < plan.code.size(); ++k) prog.code[k] = plan.code[k];
    prog.n_code = plan.code.size();
    std::vector<void*> buffers;
    auto release_all = [&] {
        for (void* b : buffers) (void)vc_hip_release(b);
    };
    for (std::size_t i = 0; i < outputs.size(); ++i) {
        void* b = nullptr;
        const int status = vc_hip_alloc((outputs[i]->size() ? outputs[i]->size() : 1) * sizeof(float), &b);
        if (status != VC_HIP_OK) {
            release_all();
            throw_status(status, "HIP allocation failed");
        }
        buffers.push_back(b);
        const unsigned char slot = static_cast<unsigned char>(plan.root_slot[roots[i]]);
        if (outputs[i]->map_expr()) {
            prog.outputs[prog.n_outputs] = static_cast<float*>(b);
            prog.output_slots[prog.n_outputs++] = slot;
        } else {
            prog.sums[prog.n_sums] = static_cast<float*>(b);
            prog.sum_slots[prog.n_sums++] = slot;
        }
    }
    if (n_sum > 0) {
        prog.rows = rows;
        prog.cols = cols;
    } else {
        prog.rows = 1;
        prog.cols = count;
    }
    const int status = count || n_sum ? vc_hip_map(&prog) : VC_HIP_OK;
    if (status != VC_HIP_OK) {
        release_all();
        throw_status(status, "HIP fused elementwise pass failed");
    }
    for (std::size_t i = 0; i < outputs.size(); ++i) outputs[i]->set_computed(buffers[i]);
}

// Per-thread state of deferred expressions: inside an ElementwiseScope?
// And the storages recorded since the scope began, for flush_elementwise.
thread_local int t_elementwise_depth = 0;
thread_local std::vector<std::weak_ptr<HipStorage>> t_pending;

std::atomic<bool>& fuse_flag() {
    static std::atomic<bool> flag{[] {
        const char* v = std::getenv("VECTORCORE_HIP_FUSE");
        return !(v && std::string(v) == "0");
    }()};
    return flag;
}

bool deferring() { return t_elementwise_depth > 0 && fuse_flag().load(); }

// The expression of an operand: its own when it is a whole pending
// expression of `count` values, otherwise an input node over its buffer
// (computed now if it is still deferred).
MapExpr operand_expr(const Storage& s, std::size_t offset, std::size_t count) {
    const auto& h = as_hip(s);
    if (offset == 0 && count == h.size())
        if (MapExpr m = h.map_expr()) return m;
    auto n = std::make_shared<MapNode>();
    n->kind = MapNode::Kind::Input;
    (void)h.ptr();
    n->input = std::const_pointer_cast<HipStorage>(h.shared_from_this());
    n->offset = offset;
    return n;
}

MapExpr constant_expr(float value) {
    auto n = std::make_shared<MapNode>();
    n->kind = MapNode::Kind::Constant;
    n->value = value;
    return n;
}

MapExpr op_expr(int op, MapExpr a, MapExpr b) {
    auto n = std::make_shared<MapNode>();
    n->op = op;
    n->a = std::move(a);
    n->b = b ? std::move(b) : n->a;
    return n;
}

// Every storage an expression reads as an input.
void expr_inputs(const MapNode& root, std::vector<std::shared_ptr<HipStorage>>& out) {
    std::unordered_map<const MapNode*, int> seen;
    std::vector<const MapNode*> order;
    collect(&root, seen, order);
    for (const MapNode* n : order)
        if (n->kind == MapNode::Kind::Input &&
            std::find(out.begin(), out.end(), n->input) == out.end())
            out.push_back(n->input);
}

std::shared_ptr<HipStorage> pending_storage(std::size_t elements, MapExpr expr, std::size_t sum_rows = 0) {
    auto out = sum_rows ? std::make_shared<HipStorage>(elements, expr, sum_rows)
                        : std::make_shared<HipStorage>(elements, expr);
    std::vector<std::shared_ptr<HipStorage>> inputs;
    expr_inputs(*expr, inputs);
    for (const auto& in : inputs) in->add_reader(out);
    t_pending.push_back(out);
    return out;
}

// A deferred elementwise operation on `count` values: build(x...) makes the
// expression from the operands' expressions. When the combined expression
// does not fit one program, the operands are computed first (from the
// largest) and become inputs.
template <typename Build>
std::shared_ptr<Storage> deferred_map(std::size_t count, std::vector<std::pair<const Storage*, std::size_t>> operands,
                                      Build build) {
    std::lock_guard<std::recursive_mutex> lock(state_mutex());
    for (std::size_t round = 0; round <= operands.size(); ++round) {
        std::vector<MapExpr> ex;
        for (const auto& [s, off] : operands) ex.push_back(operand_expr(*s, off, count));
        MapExpr e = build(ex);
        if (fits({e.get()})) return pending_storage(count, std::move(e));
        // Compute the operand expression with the most operations first.
        std::size_t worst = operands.size(), worst_ops = 0;
        for (std::size_t i = 0; i < operands.size(); ++i) {
            const MapExpr& x = ex[i];
            if (x->kind != MapNode::Kind::Op) continue;
            std::unordered_map<const MapNode*, int> seen;
            std::vector<const MapNode*> order;
            collect(x.get(), seen, order);
            if (order.size() > worst_ops) {
                worst_ops = order.size();
                worst = i;
            }
        }
        if (worst == operands.size()) break;
        (void)as_hip(*operands[worst].first).ptr();
    }
    throw std::logic_error("elementwise expression does not fit one program");
}

bool contiguous(const Shape& shape, const Strides& strides) { return strides == contiguous_strides(shape); }

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

namespace {
std::atomic<bool>& strict_item_flag() {
    static std::atomic<bool> flag{[] {
        const char* v = std::getenv("VECTORCORE_HIP_STRICT_ITEM");
        return v && std::string(v) == "1";
    }()};
    return flag;
}
}  // namespace

void HipBackend::set_strict_item(bool enable) { strict_item_flag() = enable; }
bool HipBackend::strict_item() const { return strict_item_flag(); }

void HipBackend::download(const Storage& source, std::size_t offset, float* destination, std::size_t elements) {
    if (offset + elements > source.size()) throw std::out_of_range("HIP download exceeds storage");
    const auto& h = as_hip(source);
    if (strict_item()) synchronize();
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
    if (deferring() && count > 0 && a_shape == out_shape && b_shape == out_shape && contiguous(a_shape, a_strides) &&
        contiguous(b_shape, b_strides)) {
        const int op = binary_code(operation);  // VC_MAP_ADD..VC_MAP_DIV share the binary codes
        return deferred_map(count, {{&a, a_offset}, {&b, b_offset}},
                            [op](std::vector<MapExpr>& x) { return op_expr(op, x[0], x[1]); });
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
    if (deferring() && count > 0) {
        const int op = binary_code(operation);
        return deferred_map(count, {{&a, a_offset}}, [op, s, scalar_first](std::vector<MapExpr>& x) {
            return scalar_first ? op_expr(op, constant_expr(s), x[0]) : op_expr(op, x[0], constant_expr(s));
        });
    }
    auto out = fresh(count);
    if (count == 0) return out;
    check(vc_hip_binary_scalar(dptr(a, a_offset), count, s, scalar_first ? 1 : 0, out->ptr(), binary_code(operation)),
          "HIP binary op failed");
    return out;
}

std::shared_ptr<Storage> HipBackend::unary(const Storage& input, std::size_t offset, std::size_t count,
                                           cpu::UnaryOp operation) {
    require(*this);
    if (deferring() && count > 0 &&
        (operation == cpu::UnaryOp::Negate || operation == cpu::UnaryOp::ReluGradient)) {
        const int op = operation == cpu::UnaryOp::Negate ? VC_MAP_NEG : VC_MAP_STEP;
        return deferred_map(count, {{&input, offset}},
                            [op](std::vector<MapExpr>& x) { return op_expr(op, x[0], nullptr); });
    }
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
    // The mask as the ReLU bitmask its producer kept, when it is the whole
    // storage of a layer's fused product: the same bits, 1/32 of the reads.
    const bool single = batch == 1 && a_offsets[0] == 0 && b_offsets[0] == 0;
    const uint32_t* bits = single && mask_offset == 0 ? as_hip(mask).relu_bits(m, n) : nullptr;
    if (column_sum && single) {
        auto sums = fresh(n);
        vc_hip_colsum* pending = nullptr;
        if (bits)
            check(vc_hip_matmul_relu_bits_colsum_pending(dptr(a, a_offset), dptr(b, b_offset), out->ptr(), m, k, n,
                                                         trans_a ? 1 : 0, trans_b ? 1 : 0, bits, sums->ptr(),
                                                         &pending),
                  "HIP matmul failed");
        else
            check(vc_hip_matmul_relu_mask_colsum_pending(dptr(a, a_offset), dptr(b, b_offset), out->ptr(), m, k, n,
                                                         trans_a ? 1 : 0, trans_b ? 1 : 0, dptr(mask, mask_offset),
                                                         sums->ptr(), &pending),
                  "HIP matmul failed");
        if (pending) sums->set_pending_sums(pending);
        out->set_column_sum(std::move(sums), m, n);
        return out;
    }
    if (bits) {
        check(vc_hip_matmul_relu_bits(dptr(a, a_offset), dptr(b, b_offset), out->ptr(), m, k, n, trans_a ? 1 : 0,
                                      trans_b ? 1 : 0, bits),
              "HIP matmul failed");
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
    // Row argmax the cross-entropy forward already computed from these rows.
    if (operation == cpu::ReduceOp::Argmax && inner == 1)
        if (auto indices = as_hip(input).take_row_argmax(offset, outer, length)) return indices;
    if (operation == cpu::ReduceOp::Sum && outer == 1 && offset == 0) {
        // Column sums the kernel that wrote the input already produced.
        if (auto sums = as_hip(input).take_column_sum(length, inner)) return sums;
        // Column sums of a pending expression: one more output of its program.
        if (deferring() && length > 0 && inner >= 64 && length * inner == input.size()) {
            std::lock_guard<std::recursive_mutex> lock(state_mutex());
            if (MapExpr e = as_hip(input).map_expr()) return pending_storage(inner, e, length);
        }
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
    std::vector<const vc_hip_colsum*> sums;
    std::vector<std::size_t> counts;
    for (const AxpyItem& it : items) {
        auto& t = as_hip(*it.target);
        current.push_back(t.before_write(it.target_offset, it.count));
        if (it.count == 0) continue;
        outputs.push_back(t.ptr() + it.target_offset);
        targets.push_back(current.back()->ptr() + it.target_offset);
        // A gradient that is still pending column sums (a bias gradient no
        // one has read) is finished inside the update itself.
        const vc_hip_colsum* pending = nullptr;
        if (it.source != it.target && it.source_offset == 0 && it.count == it.source->size())
            pending = as_hip(*it.source).pending_sums();
        sums.push_back(pending);
        // A source in the target's own storage (a gradient that aliases its
        // parameter, e.g. from w.backward(w)) is read from the buffer holding
        // the current contents: before_write may have given the target a
        // fresh, unwritten buffer.
        sources.push_back(pending ? nullptr
                          : it.source == it.target ? current.back()->ptr() + it.source_offset
                                                   : dptr(*it.source, it.source_offset));
        counts.push_back(it.count);
    }
    if (outputs.empty()) return;
    check(vc_hip_axpy_batch_colsum(outputs.data(), targets.data(), sources.data(), sums.data(), counts.data(),
                                   outputs.size(), alpha),
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

void HipBackend::set_fuse_elementwise(bool enable) { fuse_flag() = enable; }
bool HipBackend::fuse_elementwise() const { return fuse_flag(); }

HipBackend::ElementwiseScope::ElementwiseScope() {
    if (t_elementwise_depth++ == 0) t_pending.clear();
}
HipBackend::ElementwiseScope::~ElementwiseScope() {
    if (--t_elementwise_depth == 0) t_pending.clear();  // what is still pending is computed on first use
}

void HipBackend::flush_elementwise() {
    std::lock_guard<std::recursive_mutex> lock(state_mutex());
    std::vector<std::shared_ptr<HipStorage>> live;
    for (const auto& w : t_pending)
        if (auto p = w.lock(); p && p->map_pending()) live.push_back(std::move(p));
    t_pending.clear();
    // Groups over the same elements: a column sum with the expressions it
    // can share a pass with, then the remaining expressions, as many per
    // program as fit.
    std::vector<bool> done(live.size(), false);
    auto elements_of = [](const HipStorage& h) { return h.sum_expr() ? h.sum_rows() * h.size() : h.size(); };
    for (int sums_first = 1; sums_first >= 0; --sums_first) {
        for (std::size_t i = 0; i < live.size(); ++i) {
            if (done[i] || (sums_first != 0) != (live[i]->sum_expr() != nullptr)) continue;
            std::vector<HipStorage*> group{live[i].get()};
            std::vector<const MapNode*> roots{live[i]->sum_expr() ? live[i]->sum_expr().get() : live[i]->map_expr().get()};
            std::size_t n_out = live[i]->sum_expr() ? 0 : 1, n_sum = live[i]->sum_expr() ? 1 : 0;
            done[i] = true;
            for (std::size_t j = i + 1; j < live.size(); ++j) {
                if (done[j] || elements_of(*live[j]) != elements_of(*live[i])) continue;
                const bool sum = live[j]->sum_expr() != nullptr;
                if (sum && (n_sum == VC_HIP_MAP_SUMS || (n_sum > 0 && live[j]->size() != group[0]->size()) ||
                            (n_sum == 0)))
                    continue;
                if (!sum && n_out == VC_HIP_MAP_OUTPUTS) continue;
                roots.push_back(sum ? live[j]->sum_expr().get() : live[j]->map_expr().get());
                if (!fits(roots)) {
                    roots.pop_back();
                    continue;
                }
                group.push_back(live[j].get());
                (sum ? n_sum : n_out) += 1;
                done[j] = true;
            }
            run_maps(group);
        }
    }
}

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
    if (deferring() && count > 0) {
        // The same fp32 operations as the fused kernels below.
        return deferred_map(count, {{&grad, grad_offset}, {&saved, saved_offset}}, [kind](std::vector<MapExpr>& x) {
            switch (kind) {
                case Activation::Relu: return op_expr(VC_MAP_MUL, x[0], op_expr(VC_MAP_STEP, x[1], nullptr));
                case Activation::Sigmoid:
                    return op_expr(VC_MAP_MUL, op_expr(VC_MAP_MUL, x[0], x[1]),
                                   op_expr(VC_MAP_SUB, constant_expr(1.0F), x[1]));
                case Activation::Exp: return op_expr(VC_MAP_MUL, x[0], x[1]);
                case Activation::Log: return op_expr(VC_MAP_DIV, x[0], x[1]);
            }
            throw std::logic_error("unknown activation");
        });
    }
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
    if (deferring() && count > 0 && a_shape == out_shape && b_shape == out_shape && contiguous(a_shape, a_strides) &&
        contiguous(b_shape, b_strides)) {
        // grad / b and -(grad * a) / (b * b), as div_backward_kernel computes them.
        std::shared_ptr<Storage> da, db;
        if (need_a)
            da = deferred_map(count, {{&grad, grad_offset}, {&b, b_offset}},
                              [](std::vector<MapExpr>& x) { return op_expr(VC_MAP_DIV, x[0], x[1]); });
        if (need_b)
            db = deferred_map(count, {{&grad, grad_offset}, {&a, a_offset}, {&b, b_offset}},
                              [](std::vector<MapExpr>& x) {
                                  return op_expr(VC_MAP_DIV, op_expr(VC_MAP_NEG, op_expr(VC_MAP_MUL, x[0], x[1]), nullptr),
                                                 op_expr(VC_MAP_MUL, x[2], x[2]));
                              });
        return {da, db};
    }
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
    // The forward also leaves each row's argmax (rows floats), kept with the
    // logits for an argmax(1) of the unchanged logits: it then costs no
    // second read of them.
    auto indices = fresh(rows);
    // The loss is published as it is computed: loss.item() then waits for the
    // forward only, not the backward and update after it.
    vc_hip_mirror* published = nullptr;
    check(vc_hip_xent_forward_argmax(dptr(logits, logits_offset),
                                     reinterpret_cast<const std::int32_t*>(as_hip(targets).ptr()), rows, classes,
                                     stats->ptr(), loss->ptr(), indices->ptr(), &published),
          "HIP cross-entropy failed");
    loss->adopt_mirror(published);
    as_hip(logits).set_row_argmax(std::move(indices), logits_offset, rows, classes);
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
        vc_hip_colsum* pending = nullptr;
        check(vc_hip_xent_backward_colsum_pending(dptr(logits, logits_offset), t, as_hip(row_stats).ptr(),
                                                  seed ? nullptr : dptr(grad_loss, grad_offset), seed ? *seed : 0.0F,
                                                  rows, classes, out->ptr(), sums->ptr(), &pending),
              "HIP cross-entropy backward failed");
        if (pending) sums->set_pending_sums(pending);
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
