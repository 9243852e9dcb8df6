// Kernels of the `cpu` device. Results follow the reference CPU path's
// arithmetic (src/cpu/cpu_backend.cpp): the same fp32 operations per element,
// GEMM sums of each 256-deep k panel added into the output, double
// accumulation for sums, first-index-wins max/argmax.
#include "vectorcore/cpu_backend.hpp"

#include "parallel.hpp"

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <vector>

namespace vectorcore::cpu {

namespace {

constexpr std::size_t kGrain = std::size_t(1) << 15;
constexpr std::size_t kPanel = 256;  // k depth summed in fp32 before joining the output

template <class F>
void binary_loop(const float* a, const Shape& a_shape, const Strides& a_strides, const float* b, const Shape& b_shape,
                 const Strides& b_strides, float* out, const Shape& out_shape, F f) {
    const std::size_t count = numel(out_shape);
    if (count == 0) return;
    const std::size_t na = numel(a_shape), nb = numel(b_shape);
    if (a_shape == out_shape && b_shape == out_shape) {
        parallel_for(count, kGrain, [&](std::size_t i0, std::size_t i1) {
            for (std::size_t i = i0; i < i1; ++i) out[i] = f(a[i], b[i]);
        });
        return;
    }
    if (nb == 1 && a_shape == out_shape) {
        const float s = b[0];
        parallel_for(count, kGrain, [&](std::size_t i0, std::size_t i1) {
            for (std::size_t i = i0; i < i1; ++i) out[i] = f(a[i], s);
        });
        return;
    }
    if (na == 1 && b_shape == out_shape) {
        const float s = a[0];
        parallel_for(count, kGrain, [&](std::size_t i0, std::size_t i1) {
            for (std::size_t i = i0; i < i1; ++i) out[i] = f(s, b[i]);
        });
        return;
    }
    // General broadcast: per output row, resolve both row starts, then walk the
    // last axis with a step of 0 or the operand's last stride.
    const std::size_t rank = out_shape.size();
    const std::size_t inner = rank ? out_shape.back() : 1;
    const std::size_t rows = count / inner;
    auto step_of = [&](const Shape& s, const Strides& st) -> std::size_t {
        return (rank == 0 || s.empty() || s.back() == 1) ? 0 : st.back();
    };
    const std::size_t sa = step_of(a_shape, a_strides), sb = step_of(b_shape, b_strides);
    parallel_for(rows, std::max<std::size_t>(1, kGrain / std::max<std::size_t>(inner, 1)),
                 [&](std::size_t r0, std::size_t r1) {
                     for (std::size_t r = r0; r < r1; ++r) {
                         std::size_t rem = r, ao = 0, bo = 0;
                         for (std::size_t ax = rank ? rank - 1 : 0; ax-- > 0;) {
                             const std::size_t c = rem % out_shape[ax];
                             rem /= out_shape[ax];
                             if (ax + a_shape.size() >= rank) {
                                 const std::size_t i = ax + a_shape.size() - rank;
                                 if (a_shape[i] != 1) ao += c * a_strides[i];
                             }
                             if (ax + b_shape.size() >= rank) {
                                 const std::size_t i = ax + b_shape.size() - rank;
                                 if (b_shape[i] != 1) bo += c * b_strides[i];
                             }
                         }
                         float* o = out + r * inner;
                         for (std::size_t j = 0; j < inner; ++j) o[j] = f(a[ao + j * sa], b[bo + j * sb]);
                     }
                 });
}

template <class F>
void map(const float* in, float* out, std::size_t count, F f) {
    parallel_for(count, kGrain / 4, [&](std::size_t i0, std::size_t i1) {
        for (std::size_t i = i0; i < i1; ++i) out[i] = f(in[i]);
    });
}

}  // namespace

void binary(const float* a, const Shape& a_shape, const Strides& a_strides, const float* b, const Shape& b_shape,
            const Strides& b_strides, float* out, const Shape& out_shape, BinaryOp operation) {
    switch (operation) {
        case BinaryOp::Add:
            return binary_loop(a, a_shape, a_strides, b, b_shape, b_strides, out, out_shape,
                               [](float x, float y) { return x + y; });
        case BinaryOp::Subtract:
            return binary_loop(a, a_shape, a_strides, b, b_shape, b_strides, out, out_shape,
                               [](float x, float y) { return x - y; });
        case BinaryOp::Multiply:
            return binary_loop(a, a_shape, a_strides, b, b_shape, b_strides, out, out_shape,
                               [](float x, float y) { return x * y; });
        case BinaryOp::Divide:
            return binary_loop(a, a_shape, a_strides, b, b_shape, b_strides, out, out_shape,
                               [](float x, float y) { return x / y; });
    }
    throw std::logic_error("unknown binary operation");
}

void unary(const float* input, float* output, std::size_t count, UnaryOp operation) {
    switch (operation) {
        case UnaryOp::Negate: return map(input, output, count, [](float x) { return -x; });
        case UnaryOp::Relu: return map(input, output, count, [](float x) { return x > 0.0F ? x : 0.0F; });
        case UnaryOp::ReluGradient: return map(input, output, count, [](float x) { return x > 0.0F ? 1.0F : 0.0F; });
        case UnaryOp::Sigmoid:
            return map(input, output, count, [](float x) {
                if (x >= 0.0F) return 1.0F / (1.0F + std::exp(-x));  // no overflow for large |x|
                const float e = std::exp(x);
                return e / (1.0F + e);
            });
        case UnaryOp::Exp: return map(input, output, count, [](float x) { return std::exp(x); });
        case UnaryOp::Log: return map(input, output, count, [](float x) { return std::log(x); });
    }
    throw std::logic_error("unknown unary operation");
}

void matmul(const float* a, const float* b, float* out, std::size_t m, std::size_t k, std::size_t n, bool trans_a,
            bool trans_b) {
    std::fill(out, out + m * n, 0.0F);
    if (m == 0 || n == 0 || k == 0) return;
    // op(B) as contiguous [k][n] rows.
    std::vector<float> bt;
    const float* brow = b;
    if (trans_b) {
        bt.resize(k * n);
        for (std::size_t j = 0; j < n; ++j)
            for (std::size_t p = 0; p < k; ++p) bt[p * n + j] = b[j * k + p];
        brow = bt.data();
    }
    auto a_at = [&](std::size_t i, std::size_t p) { return trans_a ? a[p * m + i] : a[i * k + p]; };
    if (m * n * k <= std::size_t(32) * 32 * 32 || m < 4) {
        // Tiny products: accumulate straight into the output.
        for (std::size_t i = 0; i < m; ++i)
            for (std::size_t p = 0; p < k; ++p) {
                const float av = a_at(i, p);
                for (std::size_t j = 0; j < n; ++j) out[i * n + j] += av * brow[p * n + j];
            }
        return;
    }
    constexpr std::size_t kRows = 8;
    const std::size_t blocks = (m + kRows - 1) / kRows;
    parallel_for(blocks, 1, [&](std::size_t b0, std::size_t b1) {
        std::vector<float> panel(kRows * n);
        for (std::size_t blk = b0; blk < b1; ++blk) {
            const std::size_t i0 = blk * kRows, i1 = std::min(m, i0 + kRows);
            for (std::size_t p0 = 0; p0 < k; p0 += kPanel) {
                const std::size_t p1 = std::min(k, p0 + kPanel);
                std::fill(panel.begin(), panel.end(), 0.0F);
                for (std::size_t p = p0; p < p1; ++p) {
                    const float* bp = brow + p * n;
                    for (std::size_t i = i0; i < i1; ++i) {
                        const float av = a_at(i, p);
                        float* acc = panel.data() + (i - i0) * n;
                        for (std::size_t j = 0; j < n; ++j) acc[j] += av * bp[j];
                    }
                }
                for (std::size_t i = i0; i < i1; ++i) {
                    const float* acc = panel.data() + (i - i0) * n;
                    float* o = out + i * n;
                    for (std::size_t j = 0; j < n; ++j) o[j] += acc[j];
                }
            }
        }
    });
}

void transpose(const float* input, float* output, std::size_t batch, std::size_t rows, std::size_t cols) {
    constexpr std::size_t T = 32;
    const std::size_t row_tiles = (rows + T - 1) / T;
    parallel_for(batch * row_tiles, 4, [&](std::size_t w0, std::size_t w1) {
        for (std::size_t w = w0; w < w1; ++w) {
            const std::size_t z = w / row_tiles, r0 = (w % row_tiles) * T, r1 = std::min(rows, r0 + T);
            const float* src = input + z * rows * cols;
            float* dst = output + z * rows * cols;
            for (std::size_t c0 = 0; c0 < cols; c0 += T)
                for (std::size_t r = r0; r < r1; ++r)
                    for (std::size_t c = c0; c < std::min(cols, c0 + T); ++c) dst[c * rows + r] = src[r * cols + c];
        }
    });
}

float sum(const float* input, std::size_t count) {
    // 65536-element chunks, each with four double accumulators; chunk results
    // joined in chunk order, so the value is independent of the thread count.
    constexpr std::size_t kChunk = std::size_t(1) << 16;
    const std::size_t chunks = (count + kChunk - 1) / kChunk;
    std::vector<double> part(chunks, 0.0);
    parallel_for(chunks, 1, [&](std::size_t c0, std::size_t c1) {
        for (std::size_t c = c0; c < c1; ++c) {
            const std::size_t i0 = c * kChunk, i1 = std::min(count, i0 + kChunk);
            double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            std::size_t i = i0;
            for (; i + 4 <= i1; i += 4) {
                s0 += input[i];
                s1 += input[i + 1];
                s2 += input[i + 2];
                s3 += input[i + 3];
            }
            double t = s0 + s1 + s2 + s3;
            for (; i < i1; ++i) t += input[i];
            part[c] = t;
        }
    });
    double total = 0.0;
    for (double p : part) total += p;
    return static_cast<float>(total);
}

void reduce_axis(const float* input, float* output, std::size_t outer, std::size_t length, std::size_t inner,
                 ReduceOp operation) {
    if (length == 0 && operation != ReduceOp::Sum) throw std::invalid_argument("max/argmax over an empty axis is undefined");
    const std::size_t grain = std::max<std::size_t>(1, kGrain / std::max<std::size_t>(length * inner, 1));
    parallel_for(outer, grain, [&](std::size_t o0, std::size_t o1) {
        std::vector<double> acc;
        std::vector<float> best;
        std::vector<std::size_t> idx;
        for (std::size_t o = o0; o < o1; ++o) {
            const float* base = input + o * length * inner;
            float* dst = output + o * inner;
            if (operation == ReduceOp::Sum) {
                acc.assign(inner, 0.0);
                for (std::size_t a = 0; a < length; ++a)
                    for (std::size_t i = 0; i < inner; ++i) acc[i] += base[a * inner + i];
                for (std::size_t i = 0; i < inner; ++i) dst[i] = static_cast<float>(acc[i]);
                continue;
            }
            best.assign(base, base + inner);
            idx.assign(inner, 0);
            for (std::size_t a = 1; a < length; ++a)
                for (std::size_t i = 0; i < inner; ++i)
                    if (base[a * inner + i] > best[i]) {  // strict: the first maximum wins
                        best[i] = base[a * inner + i];
                        idx[i] = a;
                    }
            for (std::size_t i = 0; i < inner; ++i)
                dst[i] = operation == ReduceOp::Max ? best[i] : static_cast<float>(idx[i]);
        }
    });
}

void scatter_axis(const float* values, const float* indices, float* output, std::size_t outer, std::size_t length,
                  std::size_t inner) {
    std::fill(output, output + outer * length * inner, 0.0F);
    for (std::size_t o = 0; o < outer; ++o)
        for (std::size_t i = 0; i < inner; ++i) {
            const auto a = static_cast<std::size_t>(indices[o * inner + i]);
            output[(o * length + a) * inner + i] = values[o * inner + i];
        }
}

}  // namespace vectorcore::cpu
