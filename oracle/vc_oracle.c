/*
 * ORACLE — test infrastructure only (see vc_oracle.h).
 *
 * Plain-C restatement of the reference CPU kernels in src/cpu/cpu_backend.cpp.
 * Each function keeps the reference's per-element arithmetic order so that the
 * results are bit-identical to the reference itself; the loop structure (and
 * the OpenMP row split, which never changes per-element arithmetic) is this
 * file's own. Build with -ffp-contract=off: the reference's Release build
 * (ISO C++20, no -march) performs no fused multiply-adds on x86-64.
 */
#include "vc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static float apply_binary(int op, float a, float b) {
    switch (op) {
        case VCO_ADD: return a + b;
        case VCO_SUB: return a - b;
        case VCO_MUL: return a * b;
        default: return a / b;
    }
}

/* src/cpu/cpu_backend.cpp:29-106. The reference's same-shape, scalar and
 * row-broadcast fast paths compute the same op(a[i], b[j]) per element as the
 * general path, so one broadcast-index mapping covers all of them. Operands
 * are contiguous (the reference only creates contiguous tensors). */
void vco_binary(const float* a, const size_t* a_shape, size_t a_rank,
                const float* b, const size_t* b_shape, size_t b_rank,
                float* out, const size_t* out_shape, size_t out_rank, int op) {
    size_t count = 1;
    for (size_t i = 0; i < out_rank; ++i) count *= out_shape[i];
    if (count == 0) return;
    size_t a_str[16], b_str[16];
    size_t s = 1;
    for (size_t i = a_rank; i-- > 0;) { a_str[i] = s; s *= a_shape[i]; }
    s = 1;
    for (size_t i = b_rank; i-- > 0;) { b_str[i] = s; s *= b_shape[i]; }
    const size_t inner = out_rank == 0 ? 1 : out_shape[out_rank - 1];
    const size_t rows = count / inner;
    const size_t a_step = (out_rank == 0 || a_rank == 0 || a_shape[a_rank - 1] == 1) ? 0 : 1;
    const size_t b_step = (out_rank == 0 || b_rank == 0 || b_shape[b_rank - 1] == 1) ? 0 : 1;
#pragma omp parallel for schedule(static) if (count > (1u << 16))
    for (size_t row = 0; row < rows; ++row) {
        size_t rem = row, ao = 0, bo = 0;
        for (size_t axis = out_rank == 0 ? 0 : out_rank - 1; axis-- > 0;) {
            const size_t coord = rem % out_shape[axis];
            rem /= out_shape[axis];
            if (axis >= out_rank - a_rank) {
                const size_t ia = axis - (out_rank - a_rank);
                if (a_shape[ia] != 1) ao += coord * a_str[ia];
            }
            if (axis >= out_rank - b_rank) {
                const size_t ib = axis - (out_rank - b_rank);
                if (b_shape[ib] != 1) bo += coord * b_str[ib];
            }
        }
        float* o = out + row * inner;
        for (size_t j = 0; j < inner; ++j) o[j] = apply_binary(op, a[ao + j * a_step], b[bo + j * b_step]);
    }
}

/* src/cpu/cpu_backend.cpp:291-316; the sigmoid keeps the reference's branch
 * (:302-307) so exp never overflows. */
void vco_unary(const float* in, float* out, size_t count, int op) {
#pragma omp parallel for schedule(static) if (count > (1u << 14))
    for (size_t i = 0; i < count; ++i) {
        const float x = in[i];
        float y;
        switch (op) {
            case VCO_NEG: y = -x; break;
            case VCO_RELU: y = x > 0.0f ? x : 0.0f; break;
            case VCO_RELU_GRAD: y = x > 0.0f ? 1.0f : 0.0f; break;
            case VCO_SIGMOID:
                if (x >= 0.0f) {
                    y = 1.0f / (1.0f + expf(-x));
                } else {
                    const float e = expf(x);
                    y = e / (1.0f + e);
                }
                break;
            case VCO_EXP: y = expf(x); break;
            default: y = logf(x); break;
        }
        out[i] = y;
    }
}

/* src/cpu/cpu_backend.cpp:318-366. Per output element the reference computes:
 *  - small path (m*n*k <= 32^3 or m < 4, :325): c = sum over p in order, in fp32,
 *    accumulated straight into the zeroed output (matmul_small :262-271);
 *  - packed path: for every 256-deep panel (KC, :123) a fresh fp32 register
 *    tile sums a(i,p)*b(p,j) over the panel in order (microkernel :200-260),
 *    then the tile is added into the output (:257-259).
 * Packing, 8x12 slivers and 32x48 task tiles only move data; they do not
 * change this per-element sequence. */
void vco_matmul(const float* a, const float* b, float* out, size_t m, size_t k, size_t n,
                int trans_a, int trans_b) {
    memset(out, 0, m * n * sizeof(float));
    if (m == 0 || n == 0 || k == 0) return;
    /* op(B) as a [k][n] row-major copy (values unchanged). */
    float* bt = (float*)malloc(k * n * sizeof(float));
    for (size_t p = 0; p < k; ++p)
        for (size_t j = 0; j < n; ++j) bt[p * n + j] = trans_b ? b[j * k + p] : b[p * n + j];
    const int small_path = (m * n * k <= (size_t)32 * 32 * 32) || m < 4;
    const size_t kc_max = 256;
#pragma omp parallel
    {
        float* tile = (float*)malloc(n * sizeof(float));
#pragma omp for schedule(static)
        for (size_t i = 0; i < m; ++i) {
            float* row = out + i * n;
            if (small_path) {
                for (size_t p = 0; p < k; ++p) {
                    const float av = trans_a ? a[p * m + i] : a[i * k + p];
                    const float* brow = bt + p * n;
                    for (size_t j = 0; j < n; ++j) row[j] += av * brow[j];
                }
            } else {
                for (size_t p0 = 0; p0 < k; p0 += kc_max) {
                    const size_t p1 = p0 + kc_max < k ? p0 + kc_max : k;
                    memset(tile, 0, n * sizeof(float));
                    for (size_t p = p0; p < p1; ++p) {
                        const float av = trans_a ? a[p * m + i] : a[i * k + p];
                        const float* brow = bt + p * n;
                        for (size_t j = 0; j < n; ++j) tile[j] += av * brow[j];
                    }
                    for (size_t j = 0; j < n; ++j) row[j] += tile[j];
                }
            }
        }
        free(tile);
    }
    free(bt);
}

/* src/cpu/cpu_backend.cpp:368-390 (tiling only affects speed). */
void vco_transpose(const float* in, float* out, size_t batch, size_t rows, size_t cols) {
    for (size_t z = 0; z < batch; ++z) {
        const float* src = in + z * rows * cols;
        float* dst = out + z * rows * cols;
        for (size_t i = 0; i < rows; ++i)
            for (size_t j = 0; j < cols; ++j) dst[j * rows + i] = src[i * cols + j];
    }
}

/* src/cpu/cpu_backend.cpp:392-418: 65536-element chunks, four double
 * accumulators over groups of four, ((a0+a1)+a2)+a3, then the tail, then the
 * chunk partials added in chunk order. */
float vco_sum(const float* in, size_t count) {
    const size_t chunk = (size_t)1 << 16;
    double total = 0.0;
    for (size_t begin = 0; begin < count; begin += chunk) {
        const size_t end = begin + chunk < count ? begin + chunk : count;
        double acc0 = 0.0, acc1 = 0.0, acc2 = 0.0, acc3 = 0.0;
        size_t i = begin;
        for (; i + 4 <= end; i += 4) {
            acc0 += in[i];
            acc1 += in[i + 1];
            acc2 += in[i + 2];
            acc3 += in[i + 3];
        }
        double part = acc0 + acc1 + acc2 + acc3;
        for (; i < end; ++i) part += in[i];
        total += part;
    }
    return (float)total;
}

/* src/cpu/cpu_backend.cpp:420-460. Sum: double accumulator per output walked
 * along the axis in order. Max/argmax: start from the first element and
 * replace only on strict '>', so the first maximum wins and a NaN never
 * replaces (a NaN first element is never replaced). */
int vco_reduce_axis(const float* in, float* out, size_t outer, size_t length, size_t inner, int op) {
    if (length == 0 && op != VCO_SUM) return -1;
#pragma omp parallel for schedule(static) if (outer * length * inner > (1u << 16))
    for (size_t o = 0; o < outer; ++o) {
        const float* base = in + o * length * inner;
        float* dst = out + o * inner;
        for (size_t i = 0; i < inner; ++i) {
            if (op == VCO_SUM) {
                double t = 0.0;
                for (size_t a = 0; a < length; ++a) t += base[a * inner + i];
                dst[i] = (float)t;
            } else {
                float best = base[i];
                size_t idx = 0;
                for (size_t a = 1; a < length; ++a) {
                    const float v = base[a * inner + i];
                    if (v > best) { best = v; idx = a; }
                }
                dst[i] = op == VCO_MAX ? best : (float)idx;
            }
        }
    }
    return 0;
}

/* src/cpu/cpu_backend.cpp:462-471. */
void vco_scatter_axis(const float* values, const float* indices, float* out,
                      size_t outer, size_t length, size_t inner) {
    memset(out, 0, outer * length * inner * sizeof(float));
    for (size_t o = 0; o < outer; ++o)
        for (size_t i = 0; i < inner; ++i) {
            const size_t a = (size_t)indices[o * inner + i];
            out[(o * length + a) * inner + i] = values[o * inner + i];
        }
}

/* src/nn.cpp:70-74. */
void vco_sgd(float* param, const float* grad, size_t count, float lr) {
    for (size_t i = 0; i < count; ++i) param[i] -= lr * grad[i];
}
