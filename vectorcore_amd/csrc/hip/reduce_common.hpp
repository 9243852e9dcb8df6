// Device helpers shared by the reduction and cross-entropy kernels:
// wavefront/workgroup double sums with a fixed combine order, the first
// strict maximum of a row, the one-launch finish (the block that finishes last
// adds the blocks' partials) and the full sum (fixed chunks, then their sum in
// a fixed order, in one launch).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vchip {
namespace red {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr unsigned kBlock = 256;

__device__ inline f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }

// ---- cross-lane exchange ----------------------------------------------------
// Butterfly partners of the six steps of a wavefront all-reduce: lane ^ 1 and
// lane ^ 2 (DPP quad permutes), lane ^ 7 within 8 and lane ^ 15 within 16 (DPP
// half-row and row mirrors), lane ^ 16 (ds_swizzle) and lane ^ 32
// (ds_bpermute). After the six steps every lane holds the result.
__device__ inline int lane_id() { return int(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u))); }

template <int Step>
__device__ inline uint32_t partner(uint32_t v, int lane) {
    if constexpr (Step == 0) return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0xB1, 0xF, 0xF, false));
    else if constexpr (Step == 1) return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x4E, 0xF, 0xF, false));
    else if constexpr (Step == 2) return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x141, 0xF, 0xF, false));
    else if constexpr (Step == 3) return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x140, 0xF, 0xF, false));
    else if constexpr (Step == 4) return uint32_t(__builtin_amdgcn_ds_swizzle(int(v), 0x401F));
    else return uint32_t(__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, int(v)));
}

template <int Step>
__device__ inline double partner(double v, int lane) {
    const uint64_t bits = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = partner<Step>(uint32_t(bits), lane), hi = partner<Step>(uint32_t(bits >> 32), lane);
    return __builtin_bit_cast(double, lo | (hi << 32));
}

template <int Step>
__device__ inline float partner(float v, int lane) {
    return __builtin_bit_cast(float, partner<Step>(__builtin_bit_cast(uint32_t, v), lane));
}

template <int Step>
__device__ inline int partner(int v, int lane) {
    return int(partner<Step>(uint32_t(v), lane));
}

// Sum over the wavefront in a fixed order; every lane gets the same bits
// (each step adds two partners' values, and fp addition commutes).
__device__ inline double wave_sum(double v) {
    const int lane = lane_id();
    v += partner<0>(v, lane);
    v += partner<1>(v, lane);
    v += partner<2>(v, lane);
    v += partner<3>(v, lane);
    v += partner<4>(v, lane);
    v += partner<5>(v, lane);
    return v;
}

__device__ inline int wave_or(int v) {
    const int lane = lane_id();
    v |= partner<0>(v, lane);
    v |= partner<1>(v, lane);
    v |= partner<2>(v, lane);
    v |= partner<3>(v, lane);
    v |= partner<4>(v, lane);
    v |= partner<5>(v, lane);
    return v;
}

// ---- first strict maximum over a row ---------------------------------------
// The reference scans a row with strict `>` from element 0
// (src/cpu/cpu_backend.cpp:443-457): the first maximum wins and NaN never
// replaces the running best. A lane visiting its elements in ascending index
// order reproduces that with one compare, starting from {-inf, kNone}: NaN and
// -inf never win. Lanes then combine by (larger value, then smaller index).
// A row whose candidates were all -inf or NaN keeps kNone, which callers
// resolve to element 0, where the reference's scan stays; a NaN element 0 is
// the caller's check.
constexpr int kNone = 0x7FFFFFFF;

struct Best {
    float v;
    int i;
};

__device__ inline Best no_best() { return Best{-__builtin_huge_valf(), kNone}; }

__device__ inline void consider_ordered(Best& b, float v, int i) {
    if (v > b.v) {
        b.v = v;
        b.i = i;
    }
}

template <int Step>
__device__ inline Best combine_partner(Best b, int lane) {
    const float ov = partner<Step>(b.v, lane);
    const int oi = partner<Step>(b.i, lane);
    const bool take = ov > b.v || (ov == b.v && oi < b.i);
    return Best{take ? ov : b.v, take ? oi : b.i};
}

__device__ inline Best wave_best(Best b) {
    const int lane = lane_id();
    b = combine_partner<0>(b, lane);
    b = combine_partner<1>(b, lane);
    b = combine_partner<2>(b, lane);
    b = combine_partner<3>(b, lane);
    b = combine_partner<4>(b, lane);
    b = combine_partner<5>(b, lane);
    return b;
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

struct Identity {
    __device__ float operator()(float s) const { return s; }
};

// Sum of x[b0, b1) by one workgroup in double: thread t takes float4 t,
// t + blockDim, ... (then the scalar tail); eight loads in flight.
template <bool Vec>
__device__ inline double chunk_sum(const float* __restrict__ x, int64_t b0, int64_t b1) {
    double acc = 0.0;
    if (Vec) {  // b0 is a multiple of 4
        const int64_t v1 = b0 + (b1 - b0) / 4 * 4;
        const int64_t stride = int64_t(blockDim.x) * 4;
        int64_t a = b0 + int64_t(threadIdx.x) * 4;
        for (; a + 7 * stride < v1; a += 8 * stride) {
            f4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = ld4(x + a + u * stride);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc += double(v[u].x);
                acc += double(v[u].y);
                acc += double(v[u].z);
                acc += double(v[u].w);
            }
        }
        for (; a < v1; a += stride) {
            const f4 v = ld4(x + a);
            acc += double(v.x);
            acc += double(v.y);
            acc += double(v.z);
            acc += double(v.w);
        }
        for (int64_t t = v1 + threadIdx.x; t < b1; t += blockDim.x) acc += double(x[t]);
    } else {
        for (int64_t t = b0 + threadIdx.x; t < b1; t += blockDim.x) acc += double(x[t]);
    }
    return acc;
}

// ---- one launch: the block that finishes last adds the partials -----------
// Only wavefront 0 of a block takes part: the block's other wavefronts leave
// once its partial is formed, so the CU can start the next block while the
// count-in's round trips to device scope run. Lane 0 writes the partial with
// a device-scope store, waits for it to complete (s_waitcnt 0: a device-scope
// store is acknowledged once it is visible at device scope, so no release
// fence, and no L2 writeback, is needed), then counts the block in on its
// group's device-scope counter (groups of kDoneGroup blocks, one counter per
// 128-byte line, so the count is not one long queue on one address). The
// block that completes a group resets that counter and counts the group in on
// the top counter; the block that completes the last group reads every
// partial with device-scope loads and adds them in one fixed order (lane t
// takes blocks t, t + 64, ... in ascending order, then the wavefront's fixed
// butterfly), so the result does not depend on which block is last, and it
// resets the top counter for the next launch. Launches on the library's one
// stream never overlap, so each translation unit's counters (static, zero at
// load) serve all its one-launch kernels; the counter resets need no wait,
// since nothing later in the same launch reads them and the end of the launch
// makes them visible to the next.

// The wait that orders a block's partial stores before its counter atomic.
// The ordering in hardware comes from s_waitcnt 0, which waits until every
// store of this wave is acknowledged; an agent-scope store (sc1) is
// acknowledged only once it is visible at agent scope, and the finishing
// block reads the partials with sc1 loads, which read that coherent copy. The
// wait builtin alone does not stop the compiler from moving the relaxed
// atomics around it, so compiler-only fences (no instruction is emitted)
// keep the stores before it and the counter atomic after it.
__device__ inline void wait_stores_visible() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

constexpr unsigned kDoneGroup = 64, kDoneGroups = 64, kDoneStride = 32;
constexpr unsigned kMaxFinishBlocks = kDoneGroup * kDoneGroups;
static __device__ unsigned int g_group_done[kDoneGroups * kDoneStride];
static __device__ unsigned int g_groups_done;

// Called by the whole of wavefront 0 (and no other wavefront of the block);
// its lane 0 holds the block's partial. Every lane learns whether the block
// finished last. Grids of at most kMaxFinishBlocks blocks.
__device__ inline bool count_in(double block_partial, double* __restrict__ part) {
    int last = 0;
    if (threadIdx.x == 0) {
        __hip_atomic_store(&part[blockIdx.x], block_partial, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wait_stores_visible();
        const unsigned group = blockIdx.x / kDoneGroup, groups = (gridDim.x + kDoneGroup - 1) / kDoneGroup;
        const unsigned members = min(kDoneGroup, gridDim.x - group * kDoneGroup);
        unsigned* counter = &g_group_done[group * kDoneStride];
        if (__hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 == members) {
            __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = __hip_atomic_fetch_add(&g_groups_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 == groups;
        }
    }
    return __builtin_amdgcn_readfirstlane(last) != 0;
}

// In wavefront 0 of the block that finished last: the sum of
// part[0, gridDim.x) on every lane, in the order above, with device-scope
// (cache policy sc1 = 16) loads, 32 in flight per lane (one round for up to
// 2048 blocks: 16 measured ~1% slower on a 2048-block forward). Also resets
// the top counter.
__device__ inline double finish_partials(const double* __restrict__ part) {
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<double*>(part), short(0), int(gridDim.x * sizeof(double)), 0x00020000);
    const unsigned lane = threadIdx.x;
    double acc = 0.0;
    for (unsigned b0 = lane; b0 < gridDim.x; b0 += 32 * kWave) {
        double v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) {
            const unsigned b = b0 + u * kWave;  // past the grid: outside the descriptor, reads 0 (not added)
            v[u] = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(rp, b * 8u, 0, 16));
        }
#pragma unroll
        for (int u = 0; u < 32; ++u)
            if (b0 + u * kWave < gridDim.x) acc += v[u];
    }
    const double total = wave_sum(acc);
    if (lane == 0) __hip_atomic_store(&g_groups_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return total;
}

// The full sum in one launch (grids of at most kMaxFinishBlocks chunks, and
// at least one block: an empty input sums to 0): block b adds
// x[b*chunk, (b+1)*chunk) in double (chunk_sum, then the workgroup tree), and
// the block that finishes last adds the blocks' partials.
template <bool Vec, class Finish>
__global__ __launch_bounds__(kBlock) void sum_finish_kernel(const float* __restrict__ x, double* __restrict__ part,
                                                            float* __restrict__ out, int64_t n, int64_t chunk,
                                                            Finish finish) {
    __shared__ double lds[kBlock / kWave];
    const int64_t b0 = int64_t(blockIdx.x) * chunk, b1 = b0 + chunk < n ? b0 + chunk : n;
    const double partial = block_sum(chunk_sum<Vec>(x, b0, b1), lds);
    if (threadIdx.x >= kWave) return;  // wavefront 0 counts the block in
    if (!count_in(partial, part)) return;
    const double total = finish_partials(part);
    if (threadIdx.x == 0) out[0] = finish(float(total));
}

// ---- column sums from a producer's partial rows ---------------------------
// A kernel that writes a matrix can leave `rows` partial rows of its column
// sums (n doubles each, every row of the matrix in exactly one). The column
// sum is then added in one fixed order: "virtual wave" w of kCombineWaves
// adds the partial rows t = w, w + 16, w + 32, ... in ascending order, and the
// 16 wave sums are added in wave order, then rounded once to float. Every
// kernel that finishes such sums (column_partials_kernel, the SGD list
// kernel's combine blocks) takes them from combine_waves, so a column's sum
// has the same bits whichever kernel adds it.
constexpr int kCombineWaves = 16;

// acc[i] = the sum of virtual wave w0 + i * wstep for column col (V virtual
// waves at once, eight loads in flight per wave).
template <int V>
__device__ inline void combine_waves(const double* __restrict__ part, int64_t rows, int64_t n, int64_t col, int w0,
                                     int wstep, double (&acc)[V]) {
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0;
    for (int64_t t0 = 0; t0 < rows; t0 += 8 * kCombineWaves) {
        double v[V][8];
#pragma unroll
        for (int i = 0; i < V; ++i)
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t t = t0 + w0 + i * wstep + u * kCombineWaves;
                v[i][u] = t < rows ? part[t * n + col] : 0.0;
            }
#pragma unroll
        for (int i = 0; i < V; ++i)
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (t0 + w0 + i * wstep + u * kCombineWaves < rows) acc[i] += v[i][u];
    }
}

// out[col] = float(column sum) of `rows` partial rows: a workgroup takes 64
// columns with one wave per virtual wave.
static __global__ __launch_bounds__(64 * kCombineWaves) void column_partials_kernel(const double* __restrict__ part,
                                                                                   int64_t rows, int64_t n,
                                                                                   float* __restrict__ out) {
    __shared__ double wave_sum[kCombineWaves][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t col = int64_t(blockIdx.x) * 64 + lane;
    double acc[1] = {0.0};
    if (col < n) combine_waves<1>(part, rows, n, col, w, 0, acc);
    wave_sum[w][lane] = acc[0];
    __syncthreads();
    if (w == 0 && col < n) {
        double total = wave_sum[0][lane];
        for (int k = 1; k < kCombineWaves; ++k) total += wave_sum[k][lane];
        out[col] = float(total);
    }
}

}  // namespace red
}  // namespace vchip
