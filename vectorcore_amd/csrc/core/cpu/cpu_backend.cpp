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
    // General broadcast: each operand gets a stride per output axis (0 where
    // it is broadcast). A chunk of the flat output decodes its first index
    // once, then advances an odometer, carrying into the outer axes and
    // moving both operand offsets by their strides.
    const std::size_t rank = out_shape.size();
    std::vector<std::size_t> step_a(rank, 0), step_b(rank, 0);
    const auto place = [&](const Shape& shape, const Strides& strides, std::vector<std::size_t>& step) {
        const std::size_t lead = rank - shape.size();
        for (std::size_t d = 0; d < shape.size(); ++d)
            if (shape[d] != 1) step[lead + d] = strides[d];
    };
    place(a_shape, a_strides, step_a);
    place(b_shape, b_strides, step_b);
    parallel_for(count, kGrain, [&](std::size_t first, std::size_t last) {
        std::vector<std::size_t> digit(rank, 0);
        std::size_t oa = 0, ob = 0, rest = first;
        for (std::size_t d = rank; d-- > 0;) {
            digit[d] = rest % out_shape[d];
            rest /= out_shape[d];
            oa += digit[d] * step_a[d];
            ob += digit[d] * step_b[d];
        }
        for (std::size_t i = first; i < last; ++i) {
            out[i] = f(a[oa], b[ob]);
            for (std::size_t d = rank; d-- > 0;) {  // next index: carry into outer axes
                oa += step_a[d];
                ob += step_b[d];
                if (++digit[d] < out_shape[d]) break;
                oa -= digit[d] * step_a[d];
                ob -= digit[d] * step_b[d];
                digit[d] = 0;
            }
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

namespace {

constexpr std::size_t kSumChunk = std::size_t(1) << 16;

// One chunk of the full sum. Element i of the chunk goes to lane i % 4 while
// a whole group of four remains; the lanes are joined in lane order and the
// leftover elements added after them: the rounding of the reference's CPU
// sum (src/cpu/cpu_backend.cpp:392-418).
double chunk_sum(const float* x, std::size_t n) {
    double lane[4] = {0.0, 0.0, 0.0, 0.0};
    const std::size_t whole = n - n % 4;
    for (std::size_t g = 0; g < whole; g += 4)
        for (int l = 0; l < 4; ++l) lane[l] += x[g + l];
    double joined = ((lane[0] + lane[1]) + lane[2]) + lane[3];
    for (std::size_t i = whole; i < n; ++i) joined += x[i];
    return joined;
}

// Columns handled together by one task of an axis reduction: their running
// values stay in a stack array while the task walks the reduced axis.
constexpr std::size_t kColumnBlock = 512;

}  // namespace

float sum(const float* input, std::size_t count) {
    // Fixed 65536-element chunks, joined in chunk order: the same value for
    // any number of threads.
    const std::size_t chunks = (count + kSumChunk - 1) / kSumChunk;
    std::vector<double> chunk_total(chunks);
    parallel_for(chunks, 1, [&](std::size_t c0, std::size_t c1) {
        for (std::size_t c = c0; c < c1; ++c) {
            const std::size_t begin = c * kSumChunk;
            chunk_total[c] = chunk_sum(input + begin, std::min(kSumChunk, count - begin));
        }
    });
    double total = 0.0;
    for (std::size_t c = 0; c < chunks; ++c) total += chunk_total[c];
    return static_cast<float>(total);
}

void reduce_axis(const float* input, float* output, std::size_t outer, std::size_t length, std::size_t inner,
                 ReduceOp operation) {
    if (length == 0 && operation != ReduceOp::Sum) throw std::invalid_argument("max/argmax over an empty axis is undefined");
    // Tasks are (outer index, block of up to kColumnBlock columns), so even a
    // single outer index (a bias gradient) spreads over the threads. Every
    // output is a sequential walk along the axis from index 0, as in the
    // reference: a double sum, or the first strict maximum.
    const std::size_t blocks = (inner + kColumnBlock - 1) / kColumnBlock;
    const std::size_t work = std::max<std::size_t>(1, length * std::min(inner, kColumnBlock));
    parallel_for(outer * blocks, std::max<std::size_t>(1, kGrain / work), [&](std::size_t t0, std::size_t t1) {
        double total[kColumnBlock];
        float top[kColumnBlock];
        std::size_t where[kColumnBlock];
        for (std::size_t t = t0; t < t1; ++t) {
            const std::size_t o = t / blocks, c0 = (t % blocks) * kColumnBlock;
            const std::size_t width = std::min(kColumnBlock, inner - c0);
            const float* column = input + o * length * inner + c0;
            float* dst = output + o * inner + c0;
            if (operation == ReduceOp::Sum) {
                std::fill(total, total + width, 0.0);
                for (std::size_t a = 0; a < length; ++a, column += inner)
                    for (std::size_t j = 0; j < width; ++j) total[j] += column[j];
                for (std::size_t j = 0; j < width; ++j) dst[j] = static_cast<float>(total[j]);
                continue;
            }
            for (std::size_t j = 0; j < width; ++j) {
                top[j] = column[j];
                where[j] = 0;
            }
            for (std::size_t a = 1; a < length; ++a) {
                column += inner;
                for (std::size_t j = 0; j < width; ++j) {
                    if (!(column[j] > top[j])) continue;  // a later equal value or NaN never replaces
                    top[j] = column[j];
                    where[j] = a;
                }
            }
            for (std::size_t j = 0; j < width; ++j)
                dst[j] = operation == ReduceOp::Max ? top[j] : static_cast<float>(where[j]);
        }
    });
}

void scatter_axis(const float* values, const float* indices, float* output, std::size_t outer, std::size_t length,
                  std::size_t inner) {
    // Written as a gather: output element (o, a, i) takes the value of
    // column (o, i) when that column's index is a, else 0, so each output
    // element is written once and the pass runs in parallel.
    const std::size_t slab = length * inner;
    parallel_for(outer * length, std::max<std::size_t>(1, kGrain / std::max<std::size_t>(inner, 1)),
                 [&](std::size_t r0, std::size_t r1) {
                     for (std::size_t r = r0; r < r1; ++r) {
                         const std::size_t o = r / length, a = r % length;
                         const float* v = values + o * inner;
                         const float* idx = indices + o * inner;
                         float* dst = output + o * slab + a * inner;
                         for (std::size_t i = 0; i < inner; ++i)
                             dst[i] = static_cast<std::size_t>(idx[i]) == a ? v[i] : 0.0F;
                     }
                 });
}

}  // namespace vectorcore::cpu
