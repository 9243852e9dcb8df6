// Device helpers shared by the reduction and cross-entropy kernels:
// wavefront/workgroup double sums with a fixed combine order, and the
// two-stage full sum (fixed chunks, then one workgroup).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vchip {
namespace red {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr unsigned kBlock = 256;

__device__ inline f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }

__device__ inline double wave_sum(double v) {
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Sum over the workgroup; the result is valid in thread 0.
__device__ inline double block_sum(double v, double* lds) {
    v = wave_sum(v);
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    if (lane == 0) lds[w] = v;
    __syncthreads();
    double total = 0.0;
    if (threadIdx.x == 0)
        for (int k = 0; k < int(blockDim.x / kWave); ++k) total += lds[k];
    return total;
}

// Chunk size of the full sum: a function of n only (>= 1024 elements,
// a multiple of 1024, at most 2048 chunks).
inline int64_t sum_chunk(int64_t n) {
    int64_t chunk = (n + 2047) / 2048;
    if (chunk < 1024) chunk = 1024;
    return (chunk + 1023) / 1024 * 1024;
}

// Stage one: part[b] = sum of x[b*chunk, (b+1)*chunk) in double.
template <bool Vec>
__global__ __launch_bounds__(kBlock) void sum_partial_kernel(const float* __restrict__ x, double* __restrict__ part,
                                                             int64_t n, int64_t chunk) {
    __shared__ double lds[kBlock / kWave];
    const int64_t b0 = int64_t(blockIdx.x) * chunk, b1 = b0 + chunk < n ? b0 + chunk : n;
    double acc = 0.0;
    if (Vec) {  // b0 is a multiple of 4
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

// Stage two: out = finish(float(sum of the partials)).
template <class Finish>
__global__ __launch_bounds__(kBlock) void sum_final_kernel(const double* __restrict__ part, float* __restrict__ out,
                                                           int64_t blocks, Finish finish) {
    __shared__ double lds[kBlock / kWave];
    double acc = 0.0;
    for (int64_t b = threadIdx.x; b < blocks; b += blockDim.x) acc += part[b];
    const double total = block_sum(acc, lds);
    if (threadIdx.x == 0) out[0] = finish(float(total));
}

struct Identity {
    __device__ float operator()(float s) const { return s; }
};

}  // namespace red
}  // namespace vchip
