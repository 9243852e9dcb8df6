// Deterministic reductions (full sum, axis sum/max/argmax), scatter_axis and
// the last-two-axes transpose.
//
// Determinism: every partition (rows per wavefront, segments per column,
// blocks per full sum) is a function of the shape alone, partial results are
// combined in a fixed order, and there are no atomics. Sums accumulate in
// double, as the reference's CPU kernels do (src/cpu/cpu_backend.cpp:392-441),
// so the fp32 result nearly always equals the reference's bit for bit.
//
// Max/argmax follow the reference's sequential scan with strict '>'
// (src/cpu/cpu_backend.cpp:443-457): the first maximum wins, a NaN never
// replaces the running best, and a NaN first element is never replaced. When
// the axis is split across lanes, each part keeps the best non-NaN
// (value, index) with ties going to the smaller index, and the first element
// is checked for NaN at the end; that reproduces the scan exactly.
#include "vc_hip_internal.hpp"

#include <algorithm>
#include <limits>

namespace vchip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr unsigned kBlock = 256;
constexpr int kNone = std::numeric_limits<int>::max();  // "no candidate yet"

__device__ inline f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }

struct Best {
    float v;
    int i;
};

__device__ inline void consider(Best& b, float v, int i) {
    if (v != v) return;  // NaN never becomes the best after the first element
    if (b.i == kNone || v > b.v || (v == b.v && i < b.i)) {
        b.v = v;
        b.i = i;
    }
}

__device__ inline Best combine(Best a, Best b) {
    if (b.i == kNone) return a;
    if (a.i == kNone) return b;
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

__device__ inline double wave_sum(double v) {
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ inline Best wave_best(Best b) {
    for (int off = kWave / 2; off > 0; off >>= 1) {
        Best o{__shfl_xor(b.v, off, kWave), __shfl_xor(b.i, off, kWave)};
        b = combine(b, o);
    }
    return b;
}

// ---- rows: inner == 1, one wavefront per row -----------------------------------
// op: 0 sum, 1 max, 2 argmax.
template <int Op, bool Vec>
__global__ __launch_bounds__(kBlock) void rows_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t rows,
                                                      int64_t len) {
    const int lane = threadIdx.x % kWave;
    const int64_t waves_per_grid = int64_t(gridDim.x) * (blockDim.x / kWave);
    for (int64_t r = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave; r < rows; r += waves_per_grid) {
        const float* row = x + r * len;
        if (Op == 0) {
            double acc = 0.0;
            if (Vec) {
                for (int64_t a = int64_t(lane) * 4; a < len; a += kWave * 4) {
                    const f4 v = ld4(row + a);
                    acc += double(v.x);
                    acc += double(v.y);
                    acc += double(v.z);
                    acc += double(v.w);
                }
            } else {
                for (int64_t a = lane; a < len; a += kWave) acc += double(row[a]);
            }
            acc = wave_sum(acc);
            if (lane == 0) out[r] = float(acc);
        } else {
            Best b{0.0f, kNone};
            if (Vec) {
                for (int64_t a = int64_t(lane) * 4; a < len; a += kWave * 4) {
                    const f4 v = ld4(row + a);
                    consider(b, v.x, int(a));
                    consider(b, v.y, int(a + 1));
                    consider(b, v.z, int(a + 2));
                    consider(b, v.w, int(a + 3));
                }
            } else {
                for (int64_t a = lane; a < len; a += kWave) consider(b, row[a], int(a));
            }
            b = wave_best(b);
            if (lane == 0) {
                const float first = row[0];
                if (first != first) b = Best{first, 0};
                out[r] = Op == 1 ? b.v : float(b.i);
            }
        }
    }
}

// ---- columns: inner > 1, one thread per output, sequential along the axis -------
// Walks the axis in order exactly like the reference loop.
template <int Op>
__global__ __launch_bounds__(kBlock) void cols_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t outer,
                                                      int64_t len, int64_t inner) {
    const int64_t total = outer * inner;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
        const int64_t o = t / inner, i = t % inner;
        const float* base = x + o * len * inner + i;
        if (Op == 0) {
            double acc = 0.0;
            for (int64_t a = 0; a < len; ++a) acc += double(base[a * inner]);
            out[t] = float(acc);
        } else {
            float best = base[0];
            int64_t idx = 0;
            for (int64_t a = 1; a < len; ++a) {
                const float v = base[a * inner];
                if (v > best) {
                    best = v;
                    idx = a;
                }
            }
            out[t] = Op == 1 ? best : float(idx);
        }
    }
}

// Split columns: the axis is cut into `segs` equal segments; stage one writes a
// partial per (segment, output) and stage two combines them in segment order.
// Vec: four adjacent outputs per thread (inner % 4 == 0, aligned input).
template <bool Vec>
__global__ __launch_bounds__(kBlock) void cols_sum_partial_kernel(const float* __restrict__ x, double* __restrict__ part,
                                                                  int64_t outer, int64_t len, int64_t inner, int64_t seg_len) {
    const int64_t width = Vec ? inner / 4 : inner;
    const int64_t items = outer * width;
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t s = blockIdx.y;
    if (t >= items) return;
    const int64_t o = t / width, c = t % width;
    const int64_t a0 = s * seg_len, a1 = std::min(len, a0 + seg_len);
    if (Vec) {
        const float* base = x + o * len * inner + c * 4;
        double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
        int64_t a = a0;
        for (; a + 4 <= a1; a += 4) {  // four rows in flight per thread
            const f4 v0 = ld4(base + a * inner), v1 = ld4(base + (a + 1) * inner), v2 = ld4(base + (a + 2) * inner),
                     v3 = ld4(base + (a + 3) * inner);
            s0 += double(v0.x); s1 += double(v0.y); s2 += double(v0.z); s3 += double(v0.w);
            s0 += double(v1.x); s1 += double(v1.y); s2 += double(v1.z); s3 += double(v1.w);
            s0 += double(v2.x); s1 += double(v2.y); s2 += double(v2.z); s3 += double(v2.w);
            s0 += double(v3.x); s1 += double(v3.y); s2 += double(v3.z); s3 += double(v3.w);
        }
        for (; a < a1; ++a) {
            const f4 v = ld4(base + a * inner);
            s0 += double(v.x); s1 += double(v.y); s2 += double(v.z); s3 += double(v.w);
        }
        double* p = part + s * outer * inner + o * inner + c * 4;
        p[0] = s0;
        p[1] = s1;
        p[2] = s2;
        p[3] = s3;
    } else {
        const float* base = x + o * len * inner + c;
        double acc = 0.0;
        for (int64_t a = a0; a < a1; ++a) acc += double(base[a * inner]);
        part[s * outer * inner + o * inner + c] = acc;
    }
}

__global__ __launch_bounds__(kBlock) void cols_sum_combine_kernel(const double* __restrict__ part, float* __restrict__ out,
                                                                  int64_t total, int64_t segs) {
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    double acc = 0.0;
    for (int64_t s = 0; s < segs; ++s) acc += part[s * total + t];
    out[t] = float(acc);
}

__global__ __launch_bounds__(kBlock) void cols_best_partial_kernel(const float* __restrict__ x, float* __restrict__ pv,
                                                                   int* __restrict__ pi, int64_t outer, int64_t len,
                                                                   int64_t inner, int64_t seg_len) {
    const int64_t items = outer * inner;
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t s = blockIdx.y;
    if (t >= items) return;
    const int64_t o = t / inner, i = t % inner;
    const int64_t a0 = s * seg_len, a1 = std::min(len, a0 + seg_len);
    const float* base = x + o * len * inner + i;
    Best b{0.0f, kNone};
    for (int64_t a = a0; a < a1; ++a) consider(b, base[a * inner], int(a));
    pv[s * items + t] = b.v;
    pi[s * items + t] = b.i;
}

template <int Op>
__global__ __launch_bounds__(kBlock) void cols_best_combine_kernel(const float* __restrict__ x, const float* __restrict__ pv,
                                                                   const int* __restrict__ pi, float* __restrict__ out,
                                                                   int64_t outer, int64_t len, int64_t inner, int64_t segs) {
    const int64_t items = outer * inner;
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= items) return;
    Best b{0.0f, kNone};
    for (int64_t s = 0; s < segs; ++s) b = combine(b, Best{pv[s * items + t], pi[s * items + t]});
    const int64_t o = t / inner, i = t % inner;
    const float first = x[o * len * inner + i];
    if (first != first) b = Best{first, 0};
    out[t] = Op == 1 ? b.v : float(b.i);
}

// ---- full sum: fixed blocks of `chunk` elements, then one block ------------------
__device__ inline double block_sum(double v, double* lds) {
    v = wave_sum(v);
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    if (lane == 0) lds[w] = v;
    __syncthreads();
    double total = 0.0;
    if (threadIdx.x == 0)
        for (int k = 0; k < int(blockDim.x / kWave); ++k) total += lds[k];
    return total;  // valid in thread 0
}

template <bool Vec>
__global__ __launch_bounds__(kBlock) void sum_partial_kernel(const float* __restrict__ x, double* __restrict__ part,
                                                             int64_t n, int64_t chunk) {
    __shared__ double lds[kBlock / kWave];
    const int64_t b0 = int64_t(blockIdx.x) * chunk, b1 = std::min(n, b0 + chunk);
    double acc = 0.0;
    if (Vec) {  // b0 is a multiple of 4 (chunk is)
        const int64_t v1 = b0 + (b1 - b0) / 4 * 4;
        for (int64_t a = b0 + int64_t(threadIdx.x) * 4; a < v1; a += int64_t(blockDim.x) * 4) {
            const f4 v = ld4(x + a);
            acc += double(v.x);
            acc += double(v.y);
            acc += double(v.z);
            acc += double(v.w);
        }
        for (int64_t a = v1 + threadIdx.x; a < b1; a += blockDim.x) acc += double(x[a]);
    } else {
        for (int64_t a = b0 + threadIdx.x; a < b1; a += blockDim.x) acc += double(x[a]);
    }
    const double total = block_sum(acc, lds);
    if (threadIdx.x == 0) part[blockIdx.x] = total;
}

__global__ __launch_bounds__(kBlock) void sum_final_kernel(const double* __restrict__ part, float* __restrict__ out,
                                                           int64_t blocks) {
    __shared__ double lds[kBlock / kWave];
    double acc = 0.0;
    for (int64_t b = threadIdx.x; b < blocks; b += blockDim.x) acc += part[b];
    const double total = block_sum(acc, lds);
    if (threadIdx.x == 0) out[0] = float(total);
}

// ---- scatter_axis ---------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void scatter_kernel(const float* __restrict__ values, const float* __restrict__ indices,
                                                         float* __restrict__ out, int64_t outer, int64_t len, int64_t inner) {
    const int64_t total = outer * len * inner;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
        const int64_t i = t % inner, rest = t / inner, a = rest % len, o = rest / len;
        const int64_t src = o * inner + i;
        out[t] = int64_t(indices[src]) == a ? values[src] : 0.0f;
    }
}

// ---- transpose of the last two axes through a padded LDS tile --------------------
constexpr int kTile = 32;
__global__ __launch_bounds__(kTile * 8) void transpose_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                              int64_t batch, int64_t rows, int64_t cols) {
    __shared__ float tile[kTile][kTile + 1];
    const int64_t r0 = int64_t(blockIdx.y) * kTile, c0 = int64_t(blockIdx.x) * kTile;
    for (int64_t z = blockIdx.z; z < batch; z += gridDim.z) {
        const float* src = in + z * rows * cols;
        float* dst = out + z * rows * cols;
        for (int k = threadIdx.y; k < kTile; k += 8) {
            const int64_t r = r0 + k, c = c0 + threadIdx.x;
            if (r < rows && c < cols) tile[k][threadIdx.x] = src[r * cols + c];
        }
        __syncthreads();
        for (int k = threadIdx.y; k < kTile; k += 8) {
            const int64_t c = c0 + k, r = r0 + threadIdx.x;  // out is [cols, rows]
            if (c < cols && r < rows) dst[c * rows + r] = tile[threadIdx.x][k];
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(kBlock) void zero_kernel(float* __restrict__ out, int64_t n) {
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < n; t += stride) out[t] = 0.0f;
}

void check_i32(int64_t v, const char* what) {
    if (v > std::numeric_limits<int>::max()) fail(VC_HIP_ERR_OVERFLOW, std::string(what) + " exceeds the int32 index range");
}

}  // namespace
}  // namespace vchip

using namespace vchip;

extern "C" {

int vc_hip_reduce_sum(const float* in, size_t count, float* out) {
    return guard([&] {
        Device& d = require_device();
        if (!out) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_reduce_sum: null output");
        const int64_t n = int64_t(count);
        // Partition fixed by n: chunks of at least 8192 elements, at most 2048 chunks.
        int64_t chunk = std::max<int64_t>(8192, (n + 2047) / 2048);
        chunk = (chunk + 1023) / 1024 * 1024;
        const int64_t blocks = n == 0 ? 1 : (n + chunk - 1) / chunk;
        Scratch part(size_t(blocks) * sizeof(double));
        Profiled p("reduce_sum", double(n), 4.0 * double(n));
        if (n == 0) {
            hipLaunchKernelGGL(sum_final_kernel, dim3(1), dim3(kBlock), 0, d.stream, part.as<double>(), out, int64_t(0));
        } else {
            if (aligned16(in))
                hipLaunchKernelGGL(sum_partial_kernel<true>, dim3(unsigned(blocks)), dim3(kBlock), 0, d.stream, in,
                                   part.as<double>(), n, chunk);
            else
                hipLaunchKernelGGL(sum_partial_kernel<false>, dim3(unsigned(blocks)), dim3(kBlock), 0, d.stream, in,
                                   part.as<double>(), n, chunk);
            after_launch("reduce_sum");
            hipLaunchKernelGGL(sum_final_kernel, dim3(1), dim3(kBlock), 0, d.stream, part.as<double>(), out, blocks);
        }
        after_launch("reduce_sum");
        p.done();
    });
}

int vc_hip_reduce_axis(const float* in, float* out, size_t outer_, size_t length_, size_t inner_, int op) {
    return guard([&] {
        Device& d = require_device();
        if (op < VC_REDUCE_SUM || op > VC_REDUCE_ARGMAX) fail(VC_HIP_ERR_INVALID_ARGUMENT, "unknown reduction");
        if (length_ == 0 && op != VC_REDUCE_SUM)
            fail(VC_HIP_ERR_INVALID_ARGUMENT, "max/argmax over an empty axis is undefined");
        const int64_t outer = int64_t(outer_), len = int64_t(length_), inner = int64_t(inner_);
        const int64_t total = outer * inner;
        if (total == 0) return;
        if (len == 0) {  // sum over an empty axis is zero
            hipLaunchKernelGGL(zero_kernel, dim3(grid_1d(size_t(total), kBlock, 1024)), dim3(kBlock), 0, d.stream, out, total);
            after_launch("reduce_axis_sum");
            return;
        }
        check_i32(len, "reduction axis length");
        const char* label = op == VC_REDUCE_SUM ? "reduce_axis_sum" : op == VC_REDUCE_MAX ? "reduce_axis_max" : "reduce_axis_argmax";
        Profiled p(label, double(outer * len * inner), 4.0 * double(outer * len * inner + total));
        const int64_t target_threads = int64_t(d.cu_count) * 1024;
        if (inner == 1) {
            // One wavefront per row; rows of < 16 elements waste lanes but stay correct.
            const bool vec = len % 4 == 0 && aligned16(in);
            const unsigned grid = unsigned(std::min<int64_t>((outer + 3) / 4, int64_t(d.cu_count) * 64));
#define VC_ROWS(OP)                                                                                              \
    if (vec) hipLaunchKernelGGL((rows_kernel<OP, true>), dim3(grid), dim3(kBlock), 0, d.stream, in, out, outer, len); \
    else hipLaunchKernelGGL((rows_kernel<OP, false>), dim3(grid), dim3(kBlock), 0, d.stream, in, out, outer, len)
            if (op == VC_REDUCE_SUM) { VC_ROWS(0); }
            else if (op == VC_REDUCE_MAX) { VC_ROWS(1); }
            else { VC_ROWS(2); }
#undef VC_ROWS
            after_launch(label);
            p.done();
            return;
        }
        const bool vec = op == VC_REDUCE_SUM && inner % 4 == 0 && aligned16(in);
        const int64_t items = vec ? total / 4 : total;
        if (items >= target_threads || len < 32) {
            const unsigned grid = grid_1d(size_t(total), kBlock, unsigned(d.cu_count) * 64);
            if (op == VC_REDUCE_SUM) hipLaunchKernelGGL(cols_kernel<0>, dim3(grid), dim3(kBlock), 0, d.stream, in, out, outer, len, inner);
            else if (op == VC_REDUCE_MAX) hipLaunchKernelGGL(cols_kernel<1>, dim3(grid), dim3(kBlock), 0, d.stream, in, out, outer, len, inner);
            else hipLaunchKernelGGL(cols_kernel<2>, dim3(grid), dim3(kBlock), 0, d.stream, in, out, outer, len, inner);
            after_launch(label);
            p.done();
            return;
        }
        // Split the axis so that items * segs covers the device; segments of >= 16 rows.
        int64_t segs = std::min<int64_t>((target_threads + items - 1) / items, (len + 15) / 16);
        segs = std::max<int64_t>(1, std::min<int64_t>(segs, 1024));
        const int64_t seg_len = (len + segs - 1) / segs;
        segs = (len + seg_len - 1) / seg_len;
        const dim3 grid1(unsigned((items + kBlock - 1) / kBlock), unsigned(segs));
        const unsigned grid2 = unsigned((total + kBlock - 1) / kBlock);
        if (op == VC_REDUCE_SUM) {
            Scratch part(size_t(segs * total) * sizeof(double));
            if (vec)
                hipLaunchKernelGGL(cols_sum_partial_kernel<true>, grid1, dim3(kBlock), 0, d.stream, in, part.as<double>(), outer,
                                   len, inner, seg_len);
            else
                hipLaunchKernelGGL(cols_sum_partial_kernel<false>, grid1, dim3(kBlock), 0, d.stream, in, part.as<double>(),
                                   outer, len, inner, seg_len);
            after_launch(label);
            hipLaunchKernelGGL(cols_sum_combine_kernel, dim3(grid2), dim3(kBlock), 0, d.stream, part.as<double>(), out, total,
                               segs);
        } else {
            Scratch pv(size_t(segs * total) * sizeof(float)), pi(size_t(segs * total) * sizeof(int));
            hipLaunchKernelGGL(cols_best_partial_kernel, grid1, dim3(kBlock), 0, d.stream, in, pv.as<float>(), pi.as<int>(),
                               outer, len, inner, seg_len);
            after_launch(label);
            if (op == VC_REDUCE_MAX)
                hipLaunchKernelGGL(cols_best_combine_kernel<1>, dim3(grid2), dim3(kBlock), 0, d.stream, in, pv.as<float>(),
                                   pi.as<int>(), out, outer, len, inner, segs);
            else
                hipLaunchKernelGGL(cols_best_combine_kernel<2>, dim3(grid2), dim3(kBlock), 0, d.stream, in, pv.as<float>(),
                                   pi.as<int>(), out, outer, len, inner, segs);
        }
        after_launch(label);
        p.done();
    });
}

int vc_hip_scatter_axis(const float* values, const float* indices, float* out, size_t outer, size_t length, size_t inner) {
    return guard([&] {
        Device& d = require_device();
        const int64_t total = int64_t(outer * length * inner);
        if (total == 0) return;
        Profiled p("scatter_axis", 0.0, 4.0 * double(total + 2 * outer * inner));
        hipLaunchKernelGGL(scatter_kernel, dim3(grid_1d(size_t(total), kBlock, unsigned(d.cu_count) * 16)), dim3(kBlock), 0,
                           d.stream, values, indices, out, int64_t(outer), int64_t(length), int64_t(inner));
        after_launch("scatter_axis");
        p.done();
    });
}

int vc_hip_transpose_last2(const float* in, float* out, size_t batch, size_t rows, size_t cols) {
    return guard([&] {
        Device& d = require_device();
        if (batch * rows * cols == 0) return;
        const dim3 grid(unsigned((cols + kTile - 1) / kTile), unsigned((rows + kTile - 1) / kTile),
                        unsigned(std::min<size_t>(batch, 65535)));
        if ((rows + kTile - 1) / kTile > 65535) fail(VC_HIP_ERR_OVERFLOW, "transpose: too many rows");
        Profiled p("transpose_last2", 0.0, 8.0 * double(batch * rows * cols));
        hipLaunchKernelGGL(transpose_kernel, grid, dim3(kTile, 8), 0, d.stream, in, out, int64_t(batch), int64_t(rows),
                           int64_t(cols));
        after_launch("transpose_last2");
        p.done();
    });
}

}  // extern "C"
