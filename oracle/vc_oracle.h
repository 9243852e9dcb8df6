/*
 * ORACLE — test infrastructure only.
 *
 * A plain-C restatement of VectorCore's CPU kernels (the reference algorithm
 * for the backward-pass hot path). Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only to check or time. The
 * product (vectorcore_amd) never links or calls it.
 *
 * Every function restates one reference routine and keeps its arithmetic
 * order, so that results are bit-identical to the reference built from source
 * (oracle/_ref): fp32 products summed in fp32 per 256-deep panel for GEMM,
 * double accumulation for sums, strict '>' (first index wins) for max/argmax.
 */
#ifndef VC_ORACLE_H
#define VC_ORACLE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Operation codes in the reference's enum order (include/vectorcore/cpu_backend.hpp:9-11). */
enum { VCO_ADD = 0, VCO_SUB = 1, VCO_MUL = 2, VCO_DIV = 3 };
enum { VCO_NEG = 0, VCO_RELU = 1, VCO_SIGMOID = 2, VCO_RELU_GRAD = 3, VCO_EXP = 4, VCO_LOG = 5 };
enum { VCO_SUM = 0, VCO_MAX = 1, VCO_ARGMAX = 2 };

/* Broadcast binary op over contiguous operands (src/cpu/cpu_backend.cpp:29-106). */
void vco_binary(const float* a, const size_t* a_shape, size_t a_rank,
                const float* b, const size_t* b_shape, size_t b_rank,
                float* out, const size_t* out_shape, size_t out_rank, int op);

/* Elementwise map (src/cpu/cpu_backend.cpp:291-316). */
void vco_unary(const float* in, float* out, size_t count, int op);

/* out (m x n) = op(a) @ op(b); trans_a: a stored (k x m); trans_b: b stored (n x k)
 * (src/cpu/cpu_backend.cpp:318-366; small path :262-271, threshold :325). */
void vco_matmul(const float* a, const float* b, float* out, size_t m, size_t k, size_t n,
                int trans_a, int trans_b);

/* Swap the last two axes of [batch, rows, cols] (src/cpu/cpu_backend.cpp:368-390). */
void vco_transpose(const float* in, float* out, size_t batch, size_t rows, size_t cols);

/* Chunked double sum, chunk order combine (src/cpu/cpu_backend.cpp:392-418). */
float vco_sum(const float* in, size_t count);

/* [outer, length, inner] -> [outer, inner] (src/cpu/cpu_backend.cpp:420-460).
 * Returns 0, or -1 for max/argmax over an empty axis (the reference throws). */
int vco_reduce_axis(const float* in, float* out, size_t outer, size_t length, size_t inner, int op);

/* Inverse of argmax (src/cpu/cpu_backend.cpp:462-471). */
void vco_scatter_axis(const float* values, const float* indices, float* out,
                      size_t outer, size_t length, size_t inner);

/* p -= lr * g (src/nn.cpp:70-74; the device form target += (-lr) * g is the same value). */
void vco_sgd(float* param, const float* grad, size_t count, float lr);

#ifdef __cplusplus
}
#endif

#endif
