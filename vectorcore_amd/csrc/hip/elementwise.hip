// Elementwise kernels: fill, broadcast binary, unary, axpy and the fused
// activation gradients of the backward rules.
//
// All of them are HBM-bound. Contiguous operands are read and written as
// 16-byte vectors (global_load/store_dwordx4) in a grid-stride loop that keeps
// four independent vectors in flight per thread; the grid is capped at a few
// workgroups per CU, which measured fastest for streaming on MI355X. Results
// are computed with the same fp32 operations, in the same order, as the
// reference's CPU kernels (src/cpu/cpu_backend.cpp:24-27, 291-316); the build
// disables floating-point contraction, so no fused multiply-add changes a
// rounding.
#include "reduce_common.hpp"
#include "vc_hip_internal.hpp"

#include <algorithm>
#include <limits>
#include <string>

namespace vchip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr unsigned kBlock = 256;

__device__ inline f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ inline void st4(float* p, f4 v) { __builtin_nontemporal_store(v, reinterpret_cast<f4*>(p)); }

// ---- operation functors ------------------------------------------------------

struct AddOp { __device__ float operator()(float a, float b) const { return a + b; } };
struct SubOp { __device__ float operator()(float a, float b) const { return a - b; } };
struct MulOp { __device__ float operator()(float a, float b) const { return a * b; } };
struct DivOp { __device__ float operator()(float a, float b) const { return a / b; } };

struct NegOp { __device__ float operator()(float x) const { return -x; } };
struct ReluOp { __device__ float operator()(float x) const { return x > 0.0f ? x : 0.0f; } };
struct ReluGradOp { __device__ float operator()(float x) const { return x > 0.0f ? 1.0f : 0.0f; } };
struct SigmoidOp {
    // The branch keeps exp() from overflowing (src/cpu/cpu_backend.cpp:302-307).
    __device__ float operator()(float x) const {
        if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
        const float e = expf(x);
        return e / (1.0f + e);
    }
};
struct ExpOp { __device__ float operator()(float x) const { return expf(x); } };
struct LogOp { __device__ float operator()(float x) const { return logf(x); } };

// Binary op against a scalar held in a kernel argument.
template <class Op, bool ScalarFirst>
struct ScalarOp {
    float s;
    __device__ float operator()(float x) const { return ScalarFirst ? Op()(s, x) : Op()(x, s); }
};

struct AxpyOp {
    float alpha;
    __device__ float operator()(float t, float s) const { return t + alpha * s; }
};
// grad * relu'(x), as the reference's two kernels compute it (src/ops.cpp:398-401).
struct ReluBwdOp { __device__ float operator()(float g, float x) const { return g * (x > 0.0f ? 1.0f : 0.0f); } };
// (grad * y) * (1 - y) (src/ops.cpp:408-411).
struct SigmoidBwdOp { __device__ float operator()(float g, float y) const { return (g * y) * (1.0f - y); } };

// ---- contiguous map kernels ---------------------------------------------------

template <class F>
__device__ inline f4 apply4(F f, f4 x) { return f4{f(x.x), f(x.y), f(x.z), f(x.w)}; }
template <class F>
__device__ inline f4 apply4(F f, f4 a, f4 b) { return f4{f(a.x, b.x), f(a.y, b.y), f(a.z, b.z), f(a.w, b.w)}; }

// y[i] = f(x[i]). n4 vectors, then `tail` scalars after them.
template <class F>
__device__ inline void map1_body(const float* __restrict__ x, float* __restrict__ y, size_t n4, size_t tail, F f) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n4; i += 4 * stride) {
        f4 v0 = ld4(x + 4 * i), v1 = ld4(x + 4 * (i + stride)), v2 = ld4(x + 4 * (i + 2 * stride)),
           v3 = ld4(x + 4 * (i + 3 * stride));
        st4(y + 4 * i, apply4(f, v0));
        st4(y + 4 * (i + stride), apply4(f, v1));
        st4(y + 4 * (i + 2 * stride), apply4(f, v2));
        st4(y + 4 * (i + 3 * stride), apply4(f, v3));
    }
    for (; i < n4; i += stride) st4(y + 4 * i, apply4(f, ld4(x + 4 * i)));
    const size_t t = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t < tail) y[4 * n4 + t] = f(x[4 * n4 + t]);
}

template <class F>
__global__ __launch_bounds__(kBlock) void map1_kernel(const float* __restrict__ x, float* __restrict__ y, size_t n4,
                                                      size_t tail, F f) {
    map1_body(x, y, n4, tail, f);
}

// y[i] = x[i] op s[0] (or s[0] op x[i]) with s a one-element device operand.
template <class Op, bool ScalarFirst>
__global__ __launch_bounds__(kBlock) void scalar_operand_kernel(const float* __restrict__ x, const float* __restrict__ s,
                                                                float* __restrict__ y, size_t n4, size_t tail) {
    map1_body(x, y, n4, tail, ScalarOp<Op, ScalarFirst>{s[0]});
}

// y[i] = f(a[i], b[i]).
template <class F>
__global__ __launch_bounds__(kBlock) void map2_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                      float* __restrict__ y, size_t n4, size_t tail, F f) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n4; i += 4 * stride) {
        f4 a0 = ld4(a + 4 * i), a1 = ld4(a + 4 * (i + stride)), a2 = ld4(a + 4 * (i + 2 * stride)),
           a3 = ld4(a + 4 * (i + 3 * stride));
        f4 b0 = ld4(b + 4 * i), b1 = ld4(b + 4 * (i + stride)), b2 = ld4(b + 4 * (i + 2 * stride)),
           b3 = ld4(b + 4 * (i + 3 * stride));
        st4(y + 4 * i, apply4(f, a0, b0));
        st4(y + 4 * (i + stride), apply4(f, a1, b1));
        st4(y + 4 * (i + 2 * stride), apply4(f, a2, b2));
        st4(y + 4 * (i + 3 * stride), apply4(f, a3, b3));
    }
    for (; i < n4; i += stride) st4(y + 4 * i, apply4(f, ld4(a + 4 * i), ld4(b + 4 * i)));
    const size_t t = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t < tail) y[4 * n4 + t] = f(a[4 * n4 + t], b[4 * n4 + t]);
}

// SGD over a list of parameters in one launch: o_k = t_k + alpha * s_k for
// every tensor k (o_k == t_k in place), as the per-tensor axpy computes it.
// The tensors are laid end to end in 16-byte chunks (first[k] = chunks before
// tensor k); a thread finds its tensor by a short scan. Each tensor's last
// chunk may be partial.
//
// A tensor whose gradient is still a set of pending column sums (part[k]:
// part_rows[k] partial rows of count[k] doubles, see red::combine_waves) has
// no chunks; instead the first blocks of the grid finish those sums, 16
// columns per block, and update the tensor with them: thread t runs virtual
// wave t / 16 of the fixed order for column t % 16 (eight loads in flight,
// as red::column_partials_kernel's lanes do), and the 16 wave sums are added
// in order, so the gradient has the bits red::column_partials_kernel gives it.
// These blocks come first so that their load round trips overlap the stream;
// keeping them to one virtual wave per thread keeps the kernel's registers,
// and so the streaming blocks' occupancy, those of a plain update.
constexpr int kAxpyList = 16;
constexpr int kCombineCols = 16;
static_assert(kBlock == kCombineCols * red::kCombineWaves, "one thread per (virtual wave, column)");
struct AxpyList {
    float* o[kAxpyList];
    const float* t[kAxpyList];
    const float* s[kAxpyList];
    const double* part[kAxpyList];
    int64_t part_rows[kAxpyList];
    int64_t count[kAxpyList];
    int64_t first[kAxpyList + 1];
    int combine_first[kAxpyList + 1];  // combine blocks before tensor k
    int n;
    float alpha;
};

__global__ __launch_bounds__(kBlock) void axpy_list_kernel(AxpyList L) {
    const AxpyOp f{L.alpha};
    const int combine_blocks = L.combine_first[L.n];
    if (int(blockIdx.x) < combine_blocks) {
        __shared__ double wave_sum[red::kCombineWaves][kCombineCols];
        int k = 0;
        while (int(blockIdx.x) >= L.combine_first[k + 1]) ++k;
        const int c = int(threadIdx.x) % kCombineCols, w = int(threadIdx.x) / kCombineCols;
        const int64_t col = int64_t(int(blockIdx.x) - L.combine_first[k]) * kCombineCols + c;
        double acc[1] = {0.0};
        if (col < L.count[k]) red::combine_waves<1>(L.part[k], L.part_rows[k], L.count[k], col, w, 0, acc);
        wave_sum[w][c] = acc[0];
        __syncthreads();
        if (w == 0 && col < L.count[k]) {
            double total = wave_sum[0][c];
            for (int v = 1; v < red::kCombineWaves; ++v) total += wave_sum[v][c];
            L.o[k][col] = f(L.t[k][col], float(total));
        }
        return;
    }
    const int64_t total = L.first[L.n];
    const int64_t stride = int64_t(gridDim.x - combine_blocks) * blockDim.x;
    for (int64_t c = int64_t(blockIdx.x - combine_blocks) * blockDim.x + threadIdx.x; c < total; c += stride) {
        int k = 0;
        while (c >= L.first[k + 1]) ++k;
        const int64_t e = (c - L.first[k]) * 4;
        float* o = L.o[k] + e;
        const float* t = L.t[k] + e;
        const float* src = L.s[k] + e;
        if (e + 4 <= L.count[k]) {
            st4(o, apply4(f, ld4(t), ld4(src)));
        } else {
            for (int64_t i = 0; e + i < L.count[k]; ++i) o[i] = f(t[i], src[i]);
        }
    }
}

// Scalar fallbacks for buffers that are not 16-byte aligned.
template <class F>
__global__ __launch_bounds__(kBlock) void map1_scalar_kernel(const float* __restrict__ x, float* __restrict__ y, size_t n, F f) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = f(x[i]);
}
template <class F>
__global__ __launch_bounds__(kBlock) void map2_scalar_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                             float* __restrict__ y, size_t n, F f) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = f(a[i], b[i]);
}

__global__ __launch_bounds__(kBlock) void fill_kernel(float* __restrict__ y, size_t n, float v) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = v;
}

// ---- broadcast kernels -------------------------------------------------------

// Rank-2 broadcast over [rows, cols]: a at (r*as0 + c*as1), b likewise, with
// as1, bs1 in {0, 1}. One workgroup row-chunk per block, columns across lanes.
template <class Op, bool Vec>
__global__ __launch_bounds__(kBlock) void bcast2_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                        float* __restrict__ y, int64_t rows, int64_t cols, int64_t as0,
                                                        int64_t as1, int64_t bs0, int64_t bs1) {
    Op op;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* ar = a + r * as0;
        const float* br = b + r * bs0;
        float* yr = y + r * cols;
        if (Vec) {
            for (int64_t c = int64_t(threadIdx.x) * 4; c < cols; c += int64_t(blockDim.x) * 4) {
                const f4 av = as1 ? ld4(ar + c) : f4{ar[0], ar[0], ar[0], ar[0]};
                const f4 bv = bs1 ? ld4(br + c) : f4{br[0], br[0], br[0], br[0]};
                st4(yr + c, f4{op(av.x, bv.x), op(av.y, bv.y), op(av.z, bv.z), op(av.w, bv.w)});
            }
        } else {
            for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) yr[c] = op(ar[c * as1], br[c * bs1]);
        }
    }
}

// Any rank <= 8: per-element coordinates from the collapsed output shape.
template <class Op>
__global__ __launch_bounds__(kBlock) void bcast_general_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                               float* __restrict__ y, size_t n, Bcast m) {
    Op op;
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        size_t rem = i;
        int64_t ao = 0, bo = 0;
        for (int ax = m.rank - 1; ax >= 0; --ax) {
            const int64_t c = int64_t(rem % size_t(m.out_shape[ax]));
            rem /= size_t(m.out_shape[ax]);
            ao += c * m.a_stride[ax];
            bo += c * m.b_stride[ax];
        }
        y[i] = op(a[ao], b[bo]);
    }
}

// Division gradient over the output shape: ga = g / b, gb = -(g * a) / (b * b).
__global__ __launch_bounds__(kBlock) void div_backward_kernel(const float* __restrict__ g, const float* __restrict__ a,
                                                              const float* __restrict__ b, float* __restrict__ ga,
                                                              float* __restrict__ gb, size_t n, Bcast m) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        size_t rem = i;
        int64_t ao = 0, bo = 0;
        for (int ax = m.rank - 1; ax >= 0; --ax) {
            const int64_t c = int64_t(rem % size_t(m.out_shape[ax]));
            rem /= size_t(m.out_shape[ax]);
            ao += c * m.a_stride[ax];
            bo += c * m.b_stride[ax];
        }
        const float gv = g[i], bv = b[bo];
        if (ga) ga[i] = gv / bv;
        if (gb) {
            const float t = -(gv * a[ao]);
            gb[i] = t / (bv * bv);
        }
    }
}

// ---- host-side launch helpers ---------------------------------------------------

unsigned stream_grid(size_t items) {
    Device& d = device();
    return grid_1d(items, kBlock, static_cast<unsigned>(d.cu_count > 0 ? d.cu_count * 4 : 1024));
}

template <class F>
void launch_map1(const char* label, const float* x, float* y, size_t n, F f, double bytes_per_elem) {
    Device& d = require_device();
    if (n == 0) return;
    if (!x || !y) fail(VC_HIP_ERR_INVALID_ARGUMENT, std::string(label) + ": null buffer");
    Profiled p(label, 0.0, bytes_per_elem * double(n));
    if (aligned16(x) && aligned16(y)) {
        const size_t n4 = n / 4, tail = n % 4;
        launch(map1_kernel<F>, dim3(stream_grid(n4 ? n4 : 1)), dim3(kBlock), 0, d.stream, x, y, n4, tail, f);
    } else {
        launch(map1_scalar_kernel<F>, dim3(stream_grid(n)), dim3(kBlock), 0, d.stream, x, y, n, f);
    }
    after_launch(label);
    p.done();
}

template <class F>
void launch_map2(const char* label, const float* a, const float* b, float* y, size_t n, F f, double bytes_per_elem) {
    Device& d = require_device();
    if (n == 0) return;
    if (!a || !b || !y) fail(VC_HIP_ERR_INVALID_ARGUMENT, std::string(label) + ": null buffer");
    Profiled p(label, 0.0, bytes_per_elem * double(n));
    if (aligned16(a) && aligned16(b) && aligned16(y)) {
        const size_t n4 = n / 4, tail = n % 4;
        launch(map2_kernel<F>, dim3(stream_grid(n4 ? n4 : 1)), dim3(kBlock), 0, d.stream, a, b, y, n4, tail, f);
    } else {
        launch(map2_scalar_kernel<F>, dim3(stream_grid(n)), dim3(kBlock), 0, d.stream, a, b, y, n, f);
    }
    after_launch(label);
    p.done();
}

template <class Op>
void launch_binary(const float* a, const float* b, float* y, size_t n, const Bcast& m, const char* label) {
    Device& d = require_device();
    // Same shape: a plain map.
    if (m.rank == 1 && m.a_stride[0] == 1 && m.b_stride[0] == 1) {
        launch_map2(label, a, b, y, n, Op(), 12.0);
        return;
    }
    // One side is a single element read from the device, the other contiguous.
    if (m.rank == 1 && (m.a_stride[0] == 0) != (m.b_stride[0] == 0)) {
        const bool scalar_first = m.a_stride[0] == 0;
        const float* x = scalar_first ? b : a;
        const float* s = scalar_first ? a : b;
        if (aligned16(x) && aligned16(y)) {
            Profiled p(label, 0.0, 8.0 * double(n));
            const size_t n4 = n / 4, tail = n % 4;
            if (scalar_first)
                launch((scalar_operand_kernel<Op, true>), dim3(stream_grid(n4 ? n4 : 1)), dim3(kBlock), 0,
                                   d.stream, x, s, y, n4, tail);
            else
                launch((scalar_operand_kernel<Op, false>), dim3(stream_grid(n4 ? n4 : 1)), dim3(kBlock), 0,
                                   d.stream, x, s, y, n4, tail);
            after_launch(label);
            p.done();
            return;
        }
    }
    if (m.rank == 2 && (m.a_stride[1] == 0 || m.a_stride[1] == 1) && (m.b_stride[1] == 0 || m.b_stride[1] == 1)) {
        const int64_t rows = m.out_shape[0], cols = m.out_shape[1];
        const bool vec = cols % 4 == 0 && aligned16(y) && (m.a_stride[1] == 0 || (aligned16(a) && m.a_stride[0] % 4 == 0)) &&
                         (m.b_stride[1] == 0 || (aligned16(b) && m.b_stride[0] % 4 == 0));
        const unsigned grid = static_cast<unsigned>(std::min<int64_t>(rows, int64_t(d.cu_count) * 16));
        Profiled p(label, 0.0, 8.0 * double(n));
        if (vec)
            launch((bcast2_kernel<Op, true>), dim3(grid), dim3(kBlock), 0, d.stream, a, b, y, rows, cols,
                               m.a_stride[0], m.a_stride[1], m.b_stride[0], m.b_stride[1]);
        else
            launch((bcast2_kernel<Op, false>), dim3(grid), dim3(kBlock), 0, d.stream, a, b, y, rows, cols,
                               m.a_stride[0], m.a_stride[1], m.b_stride[0], m.b_stride[1]);
        after_launch(label);
        p.done();
        return;
    }
    Profiled p(label, 0.0, 8.0 * double(n));
    launch(bcast_general_kernel<Op>, dim3(stream_grid(n)), dim3(kBlock), 0, d.stream, a, b, y, n, m);
    after_launch(label);
    p.done();
}

size_t shape_numel(const size_t* shape, size_t rank) {
    size_t n = 1;
    for (size_t i = 0; i < rank; ++i) n *= shape[i];
    return n;
}

}  // namespace
}  // namespace vchip

using namespace vchip;

extern "C" {

int vc_hip_fill(float* out, size_t count, float value) {
    return guard([&] {
        Device& d = require_device();
        if (count == 0) return;
        Profiled p("fill", 0.0, 4.0 * double(count));
        launch(fill_kernel, dim3(stream_grid(count)), dim3(kBlock), 0, d.stream, out, count, value);
        after_launch("fill");
        p.done();
    });
}

int vc_hip_binary(const float* a, const size_t* a_shape, const size_t* a_strides, size_t a_rank, const float* b,
                  const size_t* b_shape, const size_t* b_strides, size_t b_rank, float* out, const size_t* out_shape,
                  size_t out_rank, int op) {
    return guard([&] {
        require_device();
        const size_t n = shape_numel(out_shape, out_rank);
        const Bcast m = make_bcast(a_shape, a_strides, a_rank, b_shape, b_strides, b_rank, out_shape, out_rank);
        if (n == 0) return;
        switch (op) {
            case VC_BINARY_ADD: return launch_binary<AddOp>(a, b, out, n, m, "binary_add");
            case VC_BINARY_SUBTRACT: return launch_binary<SubOp>(a, b, out, n, m, "binary_sub");
            case VC_BINARY_MULTIPLY: return launch_binary<MulOp>(a, b, out, n, m, "binary_mul");
            case VC_BINARY_DIVIDE: return launch_binary<DivOp>(a, b, out, n, m, "binary_div");
            default: fail(VC_HIP_ERR_INVALID_ARGUMENT, "unknown binary operation");
        }
    });
}

int vc_hip_binary_scalar(const float* a, size_t count, float s, int scalar_first, float* out, int op) {
    return guard([&] {
        const bool sf = scalar_first != 0;
        switch (op) {
            case VC_BINARY_ADD:
                return sf ? launch_map1("scalar_add", a, out, count, ScalarOp<AddOp, true>{s}, 8.0)
                          : launch_map1("scalar_add", a, out, count, ScalarOp<AddOp, false>{s}, 8.0);
            case VC_BINARY_SUBTRACT:
                return sf ? launch_map1("scalar_sub", a, out, count, ScalarOp<SubOp, true>{s}, 8.0)
                          : launch_map1("scalar_sub", a, out, count, ScalarOp<SubOp, false>{s}, 8.0);
            case VC_BINARY_MULTIPLY:
                return sf ? launch_map1("scalar_mul", a, out, count, ScalarOp<MulOp, true>{s}, 8.0)
                          : launch_map1("scalar_mul", a, out, count, ScalarOp<MulOp, false>{s}, 8.0);
            case VC_BINARY_DIVIDE:
                return sf ? launch_map1("scalar_div", a, out, count, ScalarOp<DivOp, true>{s}, 8.0)
                          : launch_map1("scalar_div", a, out, count, ScalarOp<DivOp, false>{s}, 8.0);
            default: fail(VC_HIP_ERR_INVALID_ARGUMENT, "unknown binary operation");
        }
    });
}

int vc_hip_unary(const float* in, float* out, size_t count, int op) {
    return guard([&] {
        switch (op) {
            case VC_UNARY_NEGATE: return launch_map1("unary_neg", in, out, count, NegOp(), 8.0);
            case VC_UNARY_RELU: return launch_map1("unary_relu", in, out, count, ReluOp(), 8.0);
            case VC_UNARY_SIGMOID: return launch_map1("unary_sigmoid", in, out, count, SigmoidOp(), 8.0);
            case VC_UNARY_RELU_GRADIENT: return launch_map1("unary_relu_grad", in, out, count, ReluGradOp(), 8.0);
            case VC_UNARY_EXP: return launch_map1("unary_exp", in, out, count, ExpOp(), 8.0);
            case VC_UNARY_LOG: return launch_map1("unary_log", in, out, count, LogOp(), 8.0);
            default: fail(VC_HIP_ERR_INVALID_ARGUMENT, "unknown unary operation");
        }
    });
}

int vc_hip_axpy(float* target, const float* source, size_t count, float alpha) {
    return guard([&] { launch_map2("axpy", target, source, target, count, AxpyOp{alpha}, 12.0); });
}

int vc_hip_axpy_batch(float* const* outputs, const float* const* targets, const float* const* sources,
                      const size_t* counts, size_t tensors, float alpha) {
    return vc_hip_axpy_batch_colsum(outputs, targets, sources, nullptr, counts, tensors, alpha);
}

int vc_hip_axpy_batch_colsum(float* const* outputs, const float* const* targets, const float* const* sources,
                             const vc_hip_colsum* const* sums, const size_t* counts, size_t tensors, float alpha) {
    return guard([&] {
        Device& d = require_device();
        if (tensors > 0 && (!outputs || !targets || !sources || !counts))
            fail(VC_HIP_ERR_INVALID_ARGUMENT, "axpy_batch: null list");
        size_t i = 0;
        while (i < tensors) {
            AxpyList L{};
            double bytes = 0.0;
            int64_t stream_chunks = 0;
            // Up to kAxpyList tensors per launch: pending column sums, and
            // 16-byte-aligned tensors; any other tensor goes through the
            // single-tensor kernel on its own.
            for (; i < tensors && L.n < kAxpyList; ++i) {
                if (counts[i] == 0) continue;
                const vc_hip_colsum* pending = sums ? sums[i] : nullptr;
                if (!outputs[i] || !targets[i] || (!pending && !sources[i]))
                    fail(VC_HIP_ERR_INVALID_ARGUMENT, "axpy_batch: null buffer");
                if (pending) {
                    if (int64_t(counts[i]) != pending->n)
                        fail(VC_HIP_ERR_INVALID_ARGUMENT, "axpy_batch: pending column sums of " +
                                                              std::to_string(pending->n) + " columns for a tensor of " +
                                                              std::to_string(counts[i]));
                    const int64_t blocks = (pending->n + kCombineCols - 1) / kCombineCols;
                    if (int64_t(L.combine_first[L.n]) + blocks > std::numeric_limits<int>::max() / 2)
                        fail(VC_HIP_ERR_OVERFLOW, "axpy_batch: too many pending columns");
                    L.part[L.n] = pending->part;
                    L.part_rows[L.n] = pending->rows;
                    L.combine_first[L.n + 1] = L.combine_first[L.n] + int(blocks);
                    L.first[L.n + 1] = L.first[L.n];
                    bytes += 8.0 * double(pending->rows * pending->n) + 8.0 * double(counts[i]);
                } else {
                    if (!aligned16(outputs[i]) || !aligned16(targets[i]) || !aligned16(sources[i])) {
                        launch_map2("axpy", targets[i], sources[i], outputs[i], counts[i], AxpyOp{alpha}, 12.0);
                        continue;
                    }
                    L.s[L.n] = sources[i];
                    L.combine_first[L.n + 1] = L.combine_first[L.n];
                    L.first[L.n + 1] = L.first[L.n] + int64_t((counts[i] + 3) / 4);
                    bytes += 12.0 * double(counts[i]);
                }
                L.o[L.n] = outputs[i];
                L.t[L.n] = targets[i];
                L.count[L.n] = int64_t(counts[i]);
                stream_chunks = L.first[L.n + 1];
                ++L.n;
            }
            if (L.n == 0) continue;
            L.alpha = alpha;
            const unsigned stream_blocks = stream_chunks ? stream_grid(size_t(stream_chunks)) : 0u;
            Profiled p("axpy", 0.0, bytes);
            launch(axpy_list_kernel, dim3(unsigned(L.combine_first[L.n]) + stream_blocks), dim3(kBlock), 0, d.stream,
                   L);
            after_launch("axpy");
            p.done();
        }
    });
}

int vc_hip_relu_backward(const float* grad, const float* input, float* out, size_t count) {
    return guard([&] { launch_map2("relu_backward", grad, input, out, count, ReluBwdOp(), 12.0); });
}

int vc_hip_sigmoid_backward(const float* grad, const float* output, float* out, size_t count) {
    return guard([&] { launch_map2("sigmoid_backward", grad, output, out, count, SigmoidBwdOp(), 12.0); });
}

int vc_hip_exp_backward(const float* grad, const float* output, float* out, size_t count) {
    return guard([&] { launch_map2("exp_backward", grad, output, out, count, MulOp(), 12.0); });
}

int vc_hip_log_backward(const float* grad, const float* input, float* out, size_t count) {
    return guard([&] { launch_map2("log_backward", grad, input, out, count, DivOp(), 12.0); });
}

int vc_hip_div_backward(const float* grad, const float* a, const size_t* a_shape, const size_t* a_strides, size_t a_rank,
                        const float* b, const size_t* b_shape, const size_t* b_strides, size_t b_rank,
                        const size_t* out_shape, size_t out_rank, float* grad_a, float* grad_b) {
    return guard([&] {
        Device& d = require_device();
        const size_t n = shape_numel(out_shape, out_rank);
        const Bcast m = make_bcast(a_shape, a_strides, a_rank, b_shape, b_strides, b_rank, out_shape, out_rank);
        if (n == 0 || (!grad_a && !grad_b)) return;
        Profiled p("div_backward", 0.0, 4.0 * double(n) * (2 + (grad_a ? 1 : 0) + (grad_b ? 1 : 0)));
        launch(div_backward_kernel, dim3(stream_grid(n)), dim3(kBlock), 0, d.stream, grad, a, b, grad_a,
                           grad_b, n, m);
        after_launch("div_backward");
        p.done();
    });
}

}  // extern "C"
