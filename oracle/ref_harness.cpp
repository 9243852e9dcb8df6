// ORACLE — test infrastructure only.
//
// C entry points over the reference VectorCore library, compiled together with
// the reference's own sources (see oracle/build_oracle.py) into
// oracle/_ref/libvc_ref.so. Tests use it to pin the C oracle (vc_oracle.c) and
// bench.py times it as the CPU baseline. Everything here calls the reference's
// public C++ API (include/vectorcore/*.hpp); no reference code is copied.
#include "vectorcore/vectorcore.hpp"
#include "vectorcore/cpu_backend.hpp"

#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <thread>
#include <vector>

using vectorcore::Shape;
using vectorcore::Tensor;

namespace {

thread_local std::string g_error;

Shape make_shape(const size_t* dims, size_t rank) { return Shape(dims, dims + rank); }

std::vector<float> copy_in(const float* p, size_t n) { return std::vector<float>(p, p + n); }

void copy_out(const Tensor& t, float* dst) {
    const auto v = t.to_vector();
    std::memcpy(dst, v.data(), v.size() * sizeof(float));
}

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

struct Mlp {
    std::vector<Tensor> weights, biases;
    Tensor x;
    std::vector<std::size_t> targets;
    std::vector<Tensor*> params() {
        std::vector<Tensor*> out;
        for (size_t i = 0; i < weights.size(); ++i) {
            out.push_back(&weights[i]);
            out.push_back(&biases[i]);
        }
        return out;
    }
    Tensor logits() const {
        Tensor h = x;
        for (size_t i = 0; i < weights.size(); ++i) {
            h = h.matmul(weights[i]) + biases[i];
            if (i + 1 < weights.size()) h = h.relu();
        }
        return h;
    }
};

}  // namespace

extern "C" {

const char* ref_last_error() { return g_error.c_str(); }
unsigned ref_hardware_threads() { return std::max(1U, std::thread::hardware_concurrency()); }

// --- raw CPU kernels (include/vectorcore/cpu_backend.hpp) -------------------
int ref_binary(const float* a, const size_t* as, size_t ar, const float* b, const size_t* bs, size_t br,
               float* out, const size_t* os, size_t orank, int op) {
    return guarded([&] {
        const Shape a_shape = make_shape(as, ar), b_shape = make_shape(bs, br), o_shape = make_shape(os, orank);
        vectorcore::cpu::binary(a, a_shape, vectorcore::contiguous_strides(a_shape), b, b_shape,
                                vectorcore::contiguous_strides(b_shape), out, o_shape,
                                static_cast<vectorcore::cpu::BinaryOp>(op));
    });
}
int ref_unary(const float* in, float* out, size_t n, int op) {
    return guarded([&] { vectorcore::cpu::unary(in, out, n, static_cast<vectorcore::cpu::UnaryOp>(op)); });
}
int ref_matmul(const float* a, const float* b, float* out, size_t m, size_t k, size_t n, int ta, int tb) {
    return guarded([&] { vectorcore::cpu::matmul(a, b, out, m, k, n, ta != 0, tb != 0); });
}
int ref_sum(const float* in, size_t n, float* out) {
    return guarded([&] { *out = vectorcore::cpu::sum(in, n); });
}
int ref_reduce_axis(const float* in, float* out, size_t outer, size_t len, size_t inner, int op) {
    return guarded([&] {
        vectorcore::cpu::reduce_axis(in, out, outer, len, inner, static_cast<vectorcore::cpu::ReduceOp>(op));
    });
}

// --- autograd-level compositions --------------------------------------------
// Batched matmul backward: (A @ B).backward(dC); writes dA [a shape], dB [b shape].
int ref_matmul_backward(const float* a, const size_t* as, size_t ar, const float* b, const size_t* bs,
                        size_t br, const float* dc, float* da, float* db) {
    return guarded([&] {
        const Shape a_shape = make_shape(as, ar), b_shape = make_shape(bs, br);
        Tensor ta(copy_in(a, vectorcore::numel(a_shape)), a_shape, true);
        Tensor tb(copy_in(b, vectorcore::numel(b_shape)), b_shape, true);
        Tensor y = ta.matmul(tb);
        y.backward(Tensor(copy_in(dc, y.numel()), y.shape()));
        copy_out(ta.grad(), da);
        copy_out(tb.grad(), db);
    });
}

// y = sigmoid(relu(x + bias)) * exp(0.1 * x); y.backward(dy) -> dx, dbias.
int ref_activation_backward(const float* x, const float* bias, const float* dy, size_t rows, size_t cols,
                            float* y_out, float* dx, float* dbias) {
    return guarded([&] {
        Tensor tx(copy_in(x, rows * cols), {rows, cols}, true);
        Tensor tb(copy_in(bias, cols), {1, cols}, true);
        Tensor y = (tx + tb).relu().sigmoid() * (tx * 0.1F).exp();
        copy_out(y, y_out);
        y.backward(Tensor(copy_in(dy, rows * cols), {rows, cols}));
        copy_out(tx.grad(), dx);
        copy_out(tb.grad(), dbias);
    });
}

// Mean softmax cross-entropy (src/nn.cpp:31-53) with its backward, plus argmax.
int ref_cross_entropy(const float* logits, const int64_t* targets, size_t rows, size_t cols, float* loss,
                      float* dlogits, float* argmax) {
    return guarded([&] {
        Tensor t(copy_in(logits, rows * cols), {rows, cols}, true);
        std::vector<std::size_t> tg(rows);
        for (size_t i = 0; i < rows; ++i) tg[i] = static_cast<std::size_t>(targets[i]);
        Tensor l = vectorcore::nn::cross_entropy(t, tg);
        *loss = l.item();
        l.backward();
        copy_out(t.grad(), dlogits);
        if (argmax) copy_out(t.detach().argmax(1), argmax);
    });
}

// Stateful MLP (x @ W + b, ReLU between layers, CE loss, SGD) for train steps.
void* ref_mlp_create(size_t layers, const size_t* dims, const float* const* weights, const float* const* biases,
                     const float* x, size_t batch, const int64_t* targets) {
    try {
        auto* m = new Mlp();
        for (size_t i = 0; i < layers; ++i) {
            Tensor w(copy_in(weights[i], dims[i] * dims[i + 1]), {dims[i], dims[i + 1]}, true);
            Tensor b(copy_in(biases[i], dims[i + 1]), {dims[i + 1]}, true);
            m->weights.push_back(w);
            m->biases.push_back(b);
        }
        m->x = Tensor(copy_in(x, batch * dims[0]), {batch, dims[0]});
        m->targets.resize(batch);
        for (size_t i = 0; i < batch; ++i) m->targets[i] = static_cast<std::size_t>(targets[i]);
        return m;
    } catch (const std::exception& e) {
        g_error = e.what();
        return nullptr;
    }
}

// One train step as in benchmarks/train_benchmark.py:43-48: forward, CE,
// backward, SGD, zero_grad, loss.item().
int ref_mlp_step(void* handle, float lr, float* loss) {
    return guarded([&] {
        auto* m = static_cast<Mlp*>(handle);
        Tensor l = vectorcore::nn::cross_entropy(m->logits(), m->targets);
        l.backward();
        auto params = m->params();
        vectorcore::nn::sgd_step(params, lr);
        vectorcore::nn::zero_grad(params);
        *loss = l.item();
    });
}

// Gradients of one forward/backward (no update), for parity of the backward.
int ref_mlp_grads(void* handle, float* loss, float* const* dweights, float* const* dbiases) {
    return guarded([&] {
        auto* m = static_cast<Mlp*>(handle);
        Tensor l = vectorcore::nn::cross_entropy(m->logits(), m->targets);
        *loss = l.item();
        l.backward();
        for (size_t i = 0; i < m->weights.size(); ++i) {
            copy_out(m->weights[i].grad(), dweights[i]);
            copy_out(m->biases[i].grad(), dbiases[i]);
        }
        auto params = m->params();
        vectorcore::nn::zero_grad(params);
    });
}

int ref_mlp_params(void* handle, float* const* weights, float* const* biases) {
    return guarded([&] {
        auto* m = static_cast<Mlp*>(handle);
        for (size_t i = 0; i < m->weights.size(); ++i) {
            copy_out(m->weights[i], weights[i]);
            copy_out(m->biases[i], biases[i]);
        }
    });
}

void ref_mlp_destroy(void* handle) { delete static_cast<Mlp*>(handle); }

}  // extern "C"
