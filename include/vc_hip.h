/*
 * vc_hip.h — C ABI of the MI355X (gfx950) backend for VectorCore.
 *
 * This is the drop-in device boundary: every entry point replaces one member
 * of the reference's device interface `MetalBackend`
 * (include/vectorcore/metal_backend.hpp:13-63, implemented in
 * src/metal/metal_backend.mm), or is a fused backward kernel that a backward
 * rule in src/ops.cpp / src/nn.cpp calls instead of a chain of those members.
 *
 * Conventions
 *  - Plain C: device buffers are `float*` (or `void*`) device addresses, sizes
 *    are element counts unless the name says bytes. No C++ or torch types.
 *  - Every function returns a status (VC_HIP_OK == 0). On failure,
 *    vc_hip_last_error() holds a message for the calling thread. The ABI never
 *    throws; the C++ wrapper maps statuses to the reference's exception types
 *    (invalid_argument, out_of_range, overflow_error, runtime_error).
 *  - Work is enqueued on one in-order HIP stream owned by the library and runs
 *    asynchronously. Only vc_hip_download() and vc_hip_synchronize() wait for
 *    the device; asynchronous device faults are reported by those two calls.
 *  - Output buffers are allocated by the caller (vc_hip_alloc) and fully
 *    written by the kernel. The library never frees memory it did not
 *    allocate.
 */
#ifndef VC_HIP_H
#define VC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
#define VC_HIP_OK 0
#define VC_HIP_ERR_INVALID_ARGUMENT 1 /* std::invalid_argument in the reference */
#define VC_HIP_ERR_OUT_OF_RANGE 2     /* std::out_of_range */
#define VC_HIP_ERR_OVERFLOW 3         /* std::overflow_error */
#define VC_HIP_ERR_RUNTIME 4          /* std::runtime_error (HIP failure, device fault) */
#define VC_HIP_ERR_UNAVAILABLE 5      /* no usable gfx950 device */
#define VC_HIP_ERR_OUT_OF_MEMORY 6

/* ---- operation codes: same order as the reference enums
 *      (include/vectorcore/cpu_backend.hpp:9-11) ------------------------- */
#define VC_BINARY_ADD 0
#define VC_BINARY_SUBTRACT 1
#define VC_BINARY_MULTIPLY 2
#define VC_BINARY_DIVIDE 3
#define VC_UNARY_NEGATE 0
#define VC_UNARY_RELU 1
#define VC_UNARY_SIGMOID 2
#define VC_UNARY_RELU_GRADIENT 3
#define VC_UNARY_EXP 4
#define VC_UNARY_LOG 5
#define VC_REDUCE_SUM 0
#define VC_REDUCE_MAX 1
#define VC_REDUCE_ARGMAX 2

/* ---- device and errors --------------------------------------------------- */
/* MetalBackend::available (metal_backend.hpp:18). Initialises on first call. */
int vc_hip_available(void);
/* MetalBackend::device_name (metal_backend.hpp:19). */
const char* vc_hip_device_name(void);
/* MetalBackend::last_error (metal_backend.hpp:20): thread-local message of
 * the last failing call on this thread, or why the device is unavailable. */
const char* vc_hip_last_error(void);
/* MetalBackend::gemm_kernel (metal_backend.hpp:22): "mfma" (matrix-core
 * tiles by shape: 256 x 256 for large products, 128 x 128, or 32 x 32 for
 * products of a few tiles, and the FMA tiles for tiny products), "simple"
 * (portable FMA tiles for every product, forced by VECTORCORE_HIP_GEMM=simple),
 * "mfma128" (128 x 128 tiles for every product), "mfma256" (256 x 256 tiles
 * for every product with 16-byte aligned rows and no batch reduction, 128 x
 * 128 for the rest), or "unavailable". The last two (also settable through
 * VECTORCORE_HIP_GEMM) exist for tests and tuning: both tile sizes give the
 * same bits for a product that neither splits along K. */
const char* vc_hip_gemm_kernel(void);
/* Selects the GEMM kernel for later calls: "mfma", "simple", "mfma128" or
 * "mfma256". The reference
 * picks its kernel once, from VECTORCORE_METAL_GEMM=tiled
 * (src/metal/metal_backend.mm:96-100), and re-runs its GEMM tests in a child
 * process to cover the portable one (tests/python/test_performance_paths.py:
 * 89-103); this setter lets one process run them on both kernels. Work
 * already enqueued keeps its kernel. VC_HIP_ERR_INVALID_ARGUMENT for any
 * other name. */
int vc_hip_set_gemm_kernel(const char* name);

/* ---- memory (stream-ordered size-class pool) ----------------------------- */
/* MetalBackend::allocate (metal_backend.hpp:23, metal_backend.mm:161-182). */
int vc_hip_alloc(size_t bytes, void** out);
/* The Metal storage destructor's release (metal_backend.mm:35, 188-191): the
 * buffer returns to the pool at once; stream order keeps queued users safe. */
int vc_hip_release(void* buffer);
/* MetalBackend::upload (metal_backend.hpp:24): copies `bytes` from host
 * memory; returns once the host memory may be reused (staged, no device wait). */
int vc_hip_upload(void* dst, const void* src, size_t bytes);
/* MetalBackend::download (metal_backend.hpp:26): waits for queued work. */
int vc_hip_download(void* dst, const void* src, size_t bytes);
/* Device-to-device copy on the library stream. */
int vc_hip_copy(void* dst, const void* src, size_t bytes);
/* A one-element value published to host memory without a full
 * synchronisation: vc_hip_mirror_scalar enqueues, in stream order, a copy of
 * *device_value into a pinned host slot and returns a handle;
 * vc_hip_mirror_read waits until the stream has reached that copy (not for
 * the work enqueued after it), fails with any error the stream has already
 * recorded, and returns the value (a fault in work still running after the
 * copy surfaces at the next vc_hip_download or vc_hip_synchronize);
 * vc_hip_mirror_release
 * returns the slot. No counterpart in the reference, whose download
 * (metal_backend.mm:198-211) waits for the whole queue: it lets loss.item()
 * return while the backward pass and the optimizer step still run. */
typedef struct vc_hip_mirror vc_hip_mirror;
int vc_hip_mirror_scalar(const float* device_value, vc_hip_mirror** out);
int vc_hip_mirror_read(vc_hip_mirror* mirror, float* value);
int vc_hip_mirror_release(vc_hip_mirror* mirror);
/* MetalBackend::synchronize (metal_backend.hpp:55): waits and reports any
 * asynchronous device error. */
int vc_hip_synchronize(void);
/* Non-waiting query of the library stream: *idle = 1 when everything enqueued
 * so far has completed (or no device was initialised), else 0. Fails with an
 * error the stream has already recorded. No counterpart in the reference; it
 * lets a caller check whether a read returned before or after the queue
 * drained (see VECTORCORE_HIP_STRICT_ITEM in the C++ wrapper). */
int vc_hip_stream_idle(int* idle);

typedef struct vc_hip_pool_stats {
    uint64_t device_allocations; /* hipMalloc calls made by the pool */
    uint64_t reuses;             /* allocations served from the free lists */
    uint64_t live_bytes;         /* bytes handed out and not yet released */
    uint64_t pooled_bytes;       /* bytes parked in the free lists */
} vc_hip_pool_stats;
int vc_hip_pool_stats_get(vc_hip_pool_stats* out);
/* Returns every parked buffer to the device (waits for queued work). */
int vc_hip_pool_trim(void);

/* ---- pending column sums ---------------------------------------------------- */
/* The column sums of a matrix, left by the kernel that wrote it as partial
 * rows of double sums (every matrix row counted in exactly one) in a pool
 * buffer the handle owns: the *_colsum_pending entry points below return one.
 * Finishing adds the partial rows in one fixed order and rounds once to
 * float; vc_hip_colsum_finish and vc_hip_axpy_batch_colsum do it with the same
 * arithmetic, so both give the same bits, and a handle may be finished any
 * number of times until released. No counterpart in the reference: a bias
 * gradient there is a separate sum_to_shape pass over its operand's gradient
 * (src/autograd.cpp:50-72, src/cpu/cpu_backend.cpp:420-441); here it costs no
 * launch of its own when the optimizer step is its only reader. */
typedef struct vc_hip_colsum vc_hip_colsum;
/* column_sum[j] (n floats) = the finished sums, enqueued on the stream. */
int vc_hip_colsum_finish(const vc_hip_colsum* sums, float* column_sum);
/* *columns = n, the number of column sums. */
int vc_hip_colsum_size(const vc_hip_colsum* sums, size_t* columns);
/* Returns the partial rows to the pool in stream order (work already
 * enqueued that reads them is unaffected). NULL is accepted. */
int vc_hip_colsum_release(vc_hip_colsum* sums);

/* ---- elementwise ----------------------------------------------------------- */
int vc_hip_fill(float* out, size_t count, float value);
/* MetalBackend::binary (metal_backend.hpp:28-31): out[i] = a[.] op b[.] with
 * broadcasting by shape/strides (rank <= 8). */
int vc_hip_binary(const float* a, const size_t* a_shape, const size_t* a_strides, size_t a_rank,
                  const float* b, const size_t* b_shape, const size_t* b_strides, size_t b_rank,
                  float* out, const size_t* out_shape, size_t out_rank, int op);
/* Binary op with one operand a host-side scalar value (the scalar tensors of
 * src/tensor.cpp:323-330), so no device scalar has to be read:
 * out = a op s (scalar_first == 0) or s op a (scalar_first != 0). */
int vc_hip_binary_scalar(const float* a, size_t count, float s, int scalar_first, float* out, int op);
/* MetalBackend::unary (metal_backend.hpp:32-33). */
int vc_hip_unary(const float* in, float* out, size_t count, int op);
/* MetalBackend::axpy_inplace (metal_backend.hpp:53-54): target += alpha * source. */
int vc_hip_axpy(float* target, const float* source, size_t count, float alpha);
/* vc_hip_axpy over a list of tensors: outputs[k][i] = targets[k][i] +
 * alpha * sources[k][i] for i < counts[k] (outputs[k] == targets[k] updates in
 * place), in as few launches as the list allows (one per 16 aligned tensors).
 * An output must not overlap another entry's buffers. The same bits as calling
 * vc_hip_axpy once per tensor. No counterpart in the reference: it serves
 * nn::sgd_step (src/nn.cpp:55-76), which applies axpy_inplace
 * (metal_backend.hpp:53-54) to each parameter in turn. */
int vc_hip_axpy_batch(float* const* outputs, const float* const* targets, const float* const* sources,
                      const size_t* counts, size_t tensors, float alpha);
/* vc_hip_axpy_batch where entry k's source may be pending column sums:
 * with sums != NULL and sums[k] != NULL, outputs[k][j] = targets[k][j] +
 * alpha * (the finished sum j of sums[k]) for j < counts[k] (which must equal
 * its column count; sources[k] is not read), the same bits as
 * vc_hip_colsum_finish into a buffer followed by vc_hip_axpy_batch. The sums
 * are finished inside the same launch (blocks that run beside the other
 * tensors' updates) and the handles stay valid. No counterpart in the
 * reference: nn::sgd_step (src/nn.cpp:55-76) applying a bias gradient that
 * was never materialised. */
int vc_hip_axpy_batch_colsum(float* const* outputs, const float* const* targets, const float* const* sources,
                             const vc_hip_colsum* const* sums, const size_t* counts, size_t tensors, float alpha);

/* Fused activation gradients (one pass each; same-shape contiguous operands).
 * relu:    out = grad * (input > 0 ? 1 : 0)         (src/ops.cpp:398-401)
 * sigmoid: out = (grad * y) * (1 - y), y the output  (src/ops.cpp:408-411)
 * exp:     out = grad * y, y the output              (src/ops.cpp:363-365)
 * log:     out = grad / input                        (src/ops.cpp:372-374) */
int vc_hip_relu_backward(const float* grad, const float* input, float* out, size_t count);
int vc_hip_sigmoid_backward(const float* grad, const float* output, float* out, size_t count);
int vc_hip_exp_backward(const float* grad, const float* output, float* out, size_t count);
int vc_hip_log_backward(const float* grad, const float* input, float* out, size_t count);
/* Division gradient before sum_to_shape (src/ops.cpp:148-154), over the
 * output shape with a and b broadcast: grad_a = grad / b,
 * grad_b = -(grad * a) / (b * b). Either output may be NULL. */
int vc_hip_div_backward(const float* grad, const float* a, const size_t* a_shape, const size_t* a_strides,
                        size_t a_rank, const float* b, const size_t* b_shape, const size_t* b_strides,
                        size_t b_rank, const size_t* out_shape, size_t out_rank, float* grad_a, float* grad_b);

/* ---- fused elementwise programs -------------------------------------------- */
/* One pass of straight-line fp32 code over same-shape contiguous buffers of
 * rows * cols elements. No counterpart in the reference: the reference runs
 * each elementwise backward rule (src/ops.cpp:98-154, 363-411), each gradient
 * accumulation (src/tensor.cpp:281-288) and each bias reduction
 * (src/autograd.cpp:50-72) as a separate pass; a chain of them becomes one
 * program here, which reads every input element once and writes only the
 * values still needed.
 *
 * Slots: inputs[j] is loaded into slot j (j < n_inputs), constants[c] is slot
 * n_inputs + c; the other slots are temporaries. Instruction word:
 * op | a << 8 | b << 16 | dst << 24, computing slot[dst] = slot[a] op slot[b]
 * in fp32 (NEG and STEP read only a: -a, and a > 0 ? 1 : 0). A slot is read
 * only after it is written, constants are never written. outputs[j] receives
 * slot output_slots[j]; sums[s] ([cols]) receives the column sums of slot
 * sum_slots[s] viewed as [rows][cols], added in double in a fixed order and
 * rounded once (the reference's reduce_axis, src/cpu/cpu_backend.cpp:420-441).
 * Each output value is the same bits as the chain of single-operation kernels
 * that the program's instructions restate. Output buffers must not overlap
 * inputs or each other. */
#define VC_HIP_MAP_SLOTS 16
#define VC_HIP_MAP_CODE 32
#define VC_HIP_MAP_INPUTS 8
#define VC_HIP_MAP_CONSTANTS 8
#define VC_HIP_MAP_OUTPUTS 4
#define VC_HIP_MAP_SUMS 2
#define VC_MAP_ADD 0
#define VC_MAP_SUB 1
#define VC_MAP_MUL 2
#define VC_MAP_DIV 3
#define VC_MAP_NEG 4
#define VC_MAP_STEP 5
typedef struct vc_hip_map_program {
    const float* inputs[VC_HIP_MAP_INPUTS];
    size_t n_inputs;
    float constants[VC_HIP_MAP_CONSTANTS];
    size_t n_constants;
    uint32_t code[VC_HIP_MAP_CODE];
    size_t n_code;
    float* outputs[VC_HIP_MAP_OUTPUTS];
    unsigned char output_slots[VC_HIP_MAP_OUTPUTS];
    size_t n_outputs;
    float* sums[VC_HIP_MAP_SUMS];
    unsigned char sum_slots[VC_HIP_MAP_SUMS];
    size_t n_sums;
    size_t rows, cols;
} vc_hip_map_program;
int vc_hip_map(const vc_hip_map_program* program);

/* ---- matrix multiply ------------------------------------------------------- */
/* MetalBackend::matmul (metal_backend.hpp:34-40): for z < batch,
 * c[z*m*n ...] = op(a + a_offsets[z]) @ op(b + b_offsets[z]); op transposes
 * when trans_* is set (a stored k x m, b stored n x k), read in place. */
int vc_hip_matmul(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                  const size_t* a_offsets, const size_t* b_offsets, size_t batch, int trans_a, int trans_b);
/* vc_hip_matmul followed by the ReLU backward rule in the same kernel:
 * c = (op(a) @ op(b)) * [mask > 0], mask laid out like c ([batch][m][n],
 * contiguous): the ReLU's input or its output, which are positive at the same
 * places. The product of the two steps is the same bits as vc_hip_matmul then
 * vc_hip_relu_backward. No counterpart in the reference: it
 * fuses src/ops.cpp:395-403 into the product (src/ops.cpp:252-260) that
 * produces the ReLU's upstream gradient, when the autograd engine finds that
 * product to be the ReLU output's only consumer. */
int vc_hip_matmul_relu_mask(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                            const size_t* a_offsets, const size_t* b_offsets, size_t batch, int trans_a, int trans_b,
                            const float* mask);
/* vc_hip_matmul_relu_mask for one product (batch 1), which also writes the
 * column sums of c: column_sum[j] = sum_i c[i][j], accumulated in double in a
 * fixed order and rounded once to float. c is the same bits as
 * vc_hip_matmul_relu_mask's. The sums come from per-tile partials in the
 * product's epilogue and one small combining pass, so c is not read again.
 * No counterpart in the reference: it serves the backward of
 * relu(x @ W + b) where the ReLU's upstream gradient comes from a product
 * (src/ops.cpp:252-260, 395-403), whose add rule (src/ops.cpp:98-109) then
 * reduces that gradient to the bias's shape with sum_to_shape
 * (src/autograd.cpp:50-72), i.e. a column sum in double (reduce_axis,
 * src/cpu/cpu_backend.cpp:420-441). k must be > 0 unless m is 0. */
int vc_hip_matmul_relu_mask_colsum(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                                   int trans_a, int trans_b, const float* mask, float* column_sum);
/* vc_hip_matmul_relu_mask_colsum whose column sums may stay pending: when the
 * product's kernel keeps per-tile partial rows (any product not split along
 * K), *pending receives a handle to them and column_sum is not written;
 * otherwise *pending is NULL and column_sum is written as
 * vc_hip_matmul_relu_mask_colsum writes it. Finishing the handle gives the
 * bits vc_hip_matmul_relu_mask_colsum writes. Serves the same rules. */
int vc_hip_matmul_relu_mask_colsum_pending(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                                           int trans_a, int trans_b, const float* mask, float* column_sum,
                                           vc_hip_colsum** pending);
/* A forward layer in one kernel: c = a @ b (+ bias[column]) (then ReLU),
 * a [m][k], b [k][n], bias [n] or null, all contiguous; relu nonzero applies
 * x > 0 ? x : 0 after the bias. The same bits as vc_hip_matmul, then the
 * row-broadcast vc_hip_binary add, then vc_hip_unary relu. k must be > 0. No
 * counterpart in the reference: it fuses the add (src/ops.cpp:98-109, as
 * nn::Linear composes it, src/nn.cpp:23) and the ReLU forward
 * (src/ops.cpp:395-397) into the product (src/ops.cpp:244-249) when the
 * runtime finds those ops applied to a product not yet computed. */
int vc_hip_matmul_bias_relu(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                            const float* bias, int relu);
/* ReLU bitmask of an m x n matrix: bit i % 32 of word relu_bits[(i / 32) * n + j]
 * stands for element (i, j); ceil(m / 32) * n words. */
/* vc_hip_matmul_bias_relu with relu on, which also writes the ReLU bitmask
 * of [c > 0] when the product runs on the kernel that can (the 256-row
 * tiles, chosen by size): *bits_written is then 1, otherwise 0 and relu_bits
 * is not written. c is the same bits either way. No counterpart in the
 * reference: the bits stand for the mask that the ReLU's backward rule
 * (src/ops.cpp:395-403) reads from the layer's output, so that the product
 * giving the ReLU's upstream gradient reads 1 bit per element instead of 32
 * (vc_hip_matmul_relu_bits). */
int vc_hip_matmul_bias_relu_bits(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                                 const float* bias, uint32_t* relu_bits, int* bits_written);
/* vc_hip_matmul_relu_mask for one product (batch 1), the mask given as a ReLU
 * bitmask (mask[i][j] > 0 exactly where its bit is set): the same bits as
 * vc_hip_matmul_relu_mask with that mask. No counterpart in the reference:
 * the fused ReLU backward of vc_hip_matmul_relu_mask (src/ops.cpp:395-403). */
int vc_hip_matmul_relu_bits(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, int trans_a,
                            int trans_b, const uint32_t* relu_bits);
/* vc_hip_matmul_relu_mask_colsum_pending with the mask given as a ReLU
 * bitmask: the same bits (c, the column sums, the handle's) as with the float
 * mask it stands for. Serves the same rules. */
int vc_hip_matmul_relu_bits_colsum_pending(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                                           int trans_a, int trans_b, const uint32_t* relu_bits, float* column_sum,
                                           vc_hip_colsum** pending);

/* Batch-reduced product for gradients of a batch-broadcast operand
 * (src/ops.cpp:252-260 followed by sum_to_shape over the batch):
 * c = sum_{z < count} op(a + z*a_stride) @ op(b + z*b_stride), one fixed order. */
int vc_hip_matmul_reduce(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                         size_t count, size_t a_stride, size_t b_stride, int trans_a, int trans_b);
/* MetalBackend::transpose_last2 (metal_backend.hpp:42-43). */
int vc_hip_transpose_last2(const float* in, float* out, size_t batch, size_t rows, size_t cols);

/* ---- reductions -------------------------------------------------------------- */
/* MetalBackend::reduce_sum (metal_backend.hpp:44-45): out[0] = sum(in),
 * accumulated in double over a shape-fixed partition (deterministic). */
int vc_hip_reduce_sum(const float* in, size_t count, float* out);
/* MetalBackend::reduce_axis (metal_backend.hpp:46-48): [outer, length, inner]
 * -> [outer, inner]. Sum accumulates in double in a shape-fixed order; max and
 * argmax return the first maximum (argmax as a float index), and a NaN first
 * element wins, as in src/cpu/cpu_backend.cpp:443-457. */
int vc_hip_reduce_axis(const float* in, float* out, size_t outer, size_t length, size_t inner, int op);
/* vc_hip_reduce_axis without any device allocation: the same kernels, the
 * same results bit for bit, with the partial results (column sums, max and
 * argmax splits) in a static 2 MiB device array (one per GPU, held until the
 * process ends) instead of pool memory. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code recorded into a HIP
 * graph, tight serving loops, harnesses that forbid allocation). 2 MiB holds
 * the column sums of up to 2^17 outputs (a [8192, 4096] bias gradient needs
 * 1 MiB) and the max/argmax splits of long axes with few outputs; a call that
 * needs more fails with VC_HIP_ERR_INVALID_ARGUMENT before launching
 * anything. Row and one-thread-per-output reductions need no partial results.
 * Calls are serialised by the library and run in order on its one stream, so
 * consecutive calls reuse the array safely; nothing in it needs to start at
 * zero. Work that overlaps on one GPU (a recorded graph replayed alongside the
 * library's stream) races on the array and on the completion counters. */
int vc_hip_reduce_axis_noalloc(const float* in, float* out, size_t outer, size_t length, size_t inner, int op);
/* MetalBackend::scatter_axis (metal_backend.hpp:49-51). */
int vc_hip_scatter_axis(const float* values, const float* indices, float* out, size_t outer, size_t length,
                        size_t inner);

/* ---- softmax cross-entropy (fused loss node for src/nn.cpp:31-53) ------------- */
/* loss[0] = -(sum_i log_softmax(logits)_i[targets_i]) / rows, with the
 * reference's composition order; row_stats[2*i] = row max, row_stats[2*i+1] =
 * sum_j exp(x_ij - max) (saved for the backward). targets are class indices
 * already checked against `classes` by the caller. */
int vc_hip_xent_forward(const float* logits, const int32_t* targets, size_t rows, size_t classes,
                        float* row_stats, float* loss);
/* vc_hip_xent_forward followed by vc_hip_mirror_scalar(loss), with one launch
 * fewer: the forward's own kernel writes the mirror's host slot when it can.
 * *mirror is then read and released like vc_hip_mirror_scalar's. The fused
 * loss node of src/nn.cpp:31-53 whose value loss.item() reads; like the
 * mirrors, no counterpart in the reference's download
 * (metal_backend.mm:198-211). */
int vc_hip_xent_forward_published(const float* logits, const int32_t* targets, size_t rows, size_t classes,
                                  float* row_stats, float* loss, vc_hip_mirror** mirror);
/* vc_hip_xent_forward (mirror NULL) or vc_hip_xent_forward_published, whose
 * kernel also writes row_argmax[i] = the index of row i's first strict
 * maximum as a float (a NaN element 0 wins): the same values as
 * vc_hip_reduce_axis(logits, row_argmax, rows, classes, 1, VC_REDUCE_ARGMAX),
 * from the rows the forward already reads. No counterpart in the reference,
 * which reads the logits again for argmax (src/ops.cpp:354-358,
 * src/cpu/cpu_backend.cpp:443-457) after the loss (src/nn.cpp:31-53). */
int vc_hip_xent_forward_argmax(const float* logits, const int32_t* targets, size_t rows, size_t classes,
                               float* row_stats, float* loss, float* row_argmax, vc_hip_mirror** mirror);
/* grad_logits = (softmax(logits) - onehot(targets)) * grad_loss[0] / rows,
 * evaluated as the reference's composed backward does. grad_loss is a device
 * scalar (the upstream gradient of the loss). */
int vc_hip_xent_backward(const float* logits, const int32_t* targets, const float* row_stats,
                         const float* grad_loss, size_t rows, size_t classes, float* grad_logits);
/* vc_hip_xent_backward with the upstream gradient passed by value. No
 * counterpart in the reference: loss.backward() seeds the loss with a host
 * value (src/tensor.cpp:244-249), which then needs no upload. */
int vc_hip_xent_backward_value(const float* logits, const int32_t* targets, const float* row_stats,
                               float grad_loss, size_t rows, size_t classes, float* grad_logits);

/* vc_hip_xent_backward (grad_loss a device scalar) or
 * vc_hip_xent_backward_value (grad_loss NULL: grad_loss_value), which also
 * writes the column sums of grad_logits: column_sum[j] = sum_i
 * grad_logits[i][j], accumulated in double in a fixed order and rounded once.
 * grad_logits has the same bits as those entry points'. No counterpart in the
 * reference: it serves a loss on logits = h @ W + b, whose add rule
 * (src/ops.cpp:98-109) reduces the logits' gradient to the bias's shape with
 * sum_to_shape (src/autograd.cpp:50-72), a column sum in double
 * (src/cpu/cpu_backend.cpp:420-441); here it comes from per-row-block
 * partials the backward kernel keeps while writing grad_logits. */
int vc_hip_xent_backward_colsum(const float* logits, const int32_t* targets, const float* row_stats,
                                const float* grad_loss, float grad_loss_value, size_t rows, size_t classes,
                                float* grad_logits, float* column_sum);
/* vc_hip_xent_backward_colsum whose column sums may stay pending (rows of at
 * most 2048 classes, whose kernel keeps one partial row per 16 rows):
 * *pending then receives the handle and column_sum is not written;
 * otherwise *pending is NULL and column_sum is written. */
int vc_hip_xent_backward_colsum_pending(const float* logits, const int32_t* targets, const float* row_stats,
                                        const float* grad_loss, float grad_loss_value, size_t rows, size_t classes,
                                        float* grad_logits, float* column_sum, vc_hip_colsum** pending);

/* ---- measurement ------------------------------------------------------------- */
/* When enabled, the kernels of each labelled entry-point call carry HIP
 * events as dispatch timestamps on the library stream (no marker packets
 * between kernels), and the call's algorithmic work (FLOPs, bytes) is
 * recorded by label. Measurement support; no counterpart in the reference. */
int vc_hip_profile_enable(int enable);
/* Restricts the profiler to the comma-separated labels (e.g.
 * "gemm_nt,gemm_tn"); NULL or "" profiles every label. */
int vc_hip_profile_labels(const char* labels);
int vc_hip_profile_reset(void);
/* Waits for the stream, then reports the number of distinct labels. */
int vc_hip_profile_count(size_t* labels);
/* Aggregate of label i: launches, summed device time (ms), summed FLOPs and
 * algorithmic HBM bytes. The label string stays valid until the next reset. */
int vc_hip_profile_entry(size_t i, const char** label, uint64_t* launches, double* milliseconds,
                         double* flops, double* bytes);

#ifdef __cplusplus
}
#endif

#endif /* VC_HIP_H */
