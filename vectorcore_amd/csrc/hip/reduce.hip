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
#include "reduce_common.hpp"
#include "vc_hip_internal.hpp"

#include <algorithm>
#include <limits>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace vchip {
namespace {

using red::f4;
using red::kBlock;
using red::kWave;
using red::ld4;

using red::Best;
using red::kNone;

// Column paths visit a segment in order but merge segments by index, so they
// keep the general rule: NaN skipped, larger value first, then smaller index.
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

// ---- rows: inner == 1, one wavefront per row -----------------------------------
// Op: 0 sum, 1 max, 2 argmax. With NV > 0 (rows of at most 256 NV elements, a
// multiple of 4) each lane loads its NV float4 at once before reducing;
// otherwise it streams. Both visit a lane's elements in the same order.
template <int Op, bool Vec, int NV>
__global__ __launch_bounds__(kBlock) void rows_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t rows,
                                                      int64_t len) {
    const int lane = threadIdx.x % kWave;
    const int64_t waves_per_grid = int64_t(gridDim.x) * (blockDim.x / kWave);
    for (int64_t r = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave; r < rows; r += waves_per_grid) {
        const float* row = x + r * len;
        f4 v[NV > 0 ? NV : 1];
        if (NV > 0) {
#pragma unroll
            for (int u = 0; u < NV; ++u) {
                const int64_t a = int64_t(lane) * 4 + int64_t(u) * kWave * 4;
                v[u] = a < len ? ld4(row + a) : f4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
        if (Op == 0) {
            double acc = 0.0;
            if (NV > 0) {
#pragma unroll
                for (int u = 0; u < NV; ++u) {
                    if (int64_t(lane) * 4 + int64_t(u) * kWave * 4 < len) {
                        acc += double(v[u].x);
                        acc += double(v[u].y);
                        acc += double(v[u].z);
                        acc += double(v[u].w);
                    }
                }
            } else if (Vec) {
                for (int64_t a = int64_t(lane) * 4; a < len; a += kWave * 4) {
                    const f4 w = ld4(row + a);
                    acc += double(w.x);
                    acc += double(w.y);
                    acc += double(w.z);
                    acc += double(w.w);
                }
            } else {
                for (int64_t a = lane; a < len; a += kWave) acc += double(row[a]);
            }
            acc = red::wave_sum(acc);
            if (lane == 0) out[r] = float(acc);
        } else {
            Best b = red::no_best();
            if (NV > 0) {
#pragma unroll
                for (int u = 0; u < NV; ++u) {
                    const int a = lane * 4 + u * kWave * 4;
                    if (a < len) {
                        red::consider_ordered(b, v[u].x, a);
                        red::consider_ordered(b, v[u].y, a + 1);
                        red::consider_ordered(b, v[u].z, a + 2);
                        red::consider_ordered(b, v[u].w, a + 3);
                    }
                }
            } else if (Vec) {
                for (int64_t a = int64_t(lane) * 4; a < len; a += kWave * 4) {
                    const f4 w = ld4(row + a);
                    red::consider_ordered(b, w.x, int(a));
                    red::consider_ordered(b, w.y, int(a + 1));
                    red::consider_ordered(b, w.z, int(a + 2));
                    red::consider_ordered(b, w.w, int(a + 3));
                }
            } else {
                for (int64_t a = lane; a < len; a += kWave) red::consider_ordered(b, row[a], int(a));
            }
            b = red::wave_best(b);
            if (lane == 0) {
                const float first = NV > 0 ? v[0].x : row[0];
                if (first != first) b = Best{first, 0};
                if (b.i == kNone) b.i = 0;
                out[r] = Op == 1 ? b.v : float(b.i);
            }
        }
    }
}

// ---- columns: inner > 1, one thread per output, sequential along the axis -------
// Walks the axis in order exactly like the reference loop; used when there
// are enough outputs to fill the device.
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

// ---- tiled column sums (few outputs, long axis: bias gradients) -------------------
// Block (chunk, outer o, segment s): 16 column lanes x 16 row lanes. Column
// lane c owns 4 adjacent columns (Vec) or 1; row lane r walks rows
// a0 + r, a0 + r + 16, ... of the segment, sixteen rows in flight. A wave
// holds four row lanes of the same columns (lanes c, c + 16, c + 32, c + 48):
// they are joined with two exchanges (lane ^ 16, then lane ^ 32), then the
// four waves in wave order through LDS. One partial per (segment, column);
// with a single segment (Direct), the sum itself, rounded to float, in out.
constexpr int kColLanes = 16, kRowLanes = 16, kColInFlight = 16;

template <bool Vec, bool Direct>
__global__ __launch_bounds__(kBlock) void colsum_tile_kernel(const float* __restrict__ x, double* __restrict__ part,
                                                             float* __restrict__ out, int64_t outer, int64_t len,
                                                             int64_t inner, int64_t seg_len, int64_t chunks) {
    constexpr int W = Vec ? 4 : 1;
    constexpr int kWaves = kBlock / kWave;
    __shared__ double lds[kWaves][kColLanes * W];
    const int c = threadIdx.x % kColLanes, rl = threadIdx.x / kColLanes;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int64_t chunk = blockIdx.x % chunks, o = blockIdx.x / chunks;
    const int64_t s = blockIdx.y;
    const int64_t col = (chunk * kColLanes + c) * W;
    const int64_t a0 = s * seg_len, a1 = std::min(len, a0 + seg_len);
    double acc[W];
#pragma unroll
    for (int w = 0; w < W; ++w) acc[w] = 0.0;
    if (col < inner) {
        const float* base = x + o * len * inner + col;
        int64_t a = a0 + rl;
        for (; a + (kColInFlight - 1) * kRowLanes < a1; a += kColInFlight * kRowLanes) {
            if constexpr (Vec) {
                f4 v[kColInFlight];
#pragma unroll
                for (int u = 0; u < kColInFlight; ++u) v[u] = ld4(base + (a + u * kRowLanes) * inner);
#pragma unroll
                for (int u = 0; u < kColInFlight; ++u) {
                    acc[0] += double(v[u].x); acc[1] += double(v[u].y); acc[2] += double(v[u].z); acc[3] += double(v[u].w);
                }
            } else {
                float v[kColInFlight];
#pragma unroll
                for (int u = 0; u < kColInFlight; ++u) v[u] = base[(a + u * kRowLanes) * inner];
#pragma unroll
                for (int u = 0; u < kColInFlight; ++u) acc[0] += double(v[u]);
            }
        }
        for (; a < a1; a += kRowLanes) {
            if constexpr (Vec) {
                const f4 v = ld4(base + a * inner);
                acc[0] += double(v.x); acc[1] += double(v.y); acc[2] += double(v.z); acc[3] += double(v.w);
            } else {
                acc[0] += double(base[a * inner]);
            }
        }
    }
#pragma unroll
    for (int w = 0; w < W; ++w) {
        acc[w] += __shfl_xor(acc[w], 16, kWave);
        acc[w] += __shfl_xor(acc[w], 32, kWave);
    }
    if (lane < kColLanes) {
#pragma unroll
        for (int w = 0; w < W; ++w) lds[wave][c * W + w] = acc[w];
    }
    __syncthreads();
    if (wave == 0 && lane < kColLanes) {
#pragma unroll
        for (int w = 0; w < W; ++w) {
            double total = lds[0][c * W + w];
#pragma unroll
            for (int k = 1; k < kWaves; ++k) total += lds[k][c * W + w];
            if (col + w < inner) {
                if constexpr (Direct) out[o * inner + col + w] = float(total);
                else part[(s * outer + o) * inner + col + w] = total;
            }
        }
    }
}

// A column sum (one matrix, outer 1) in one launch. Block (chunk, segment)
// sums its 16 W columns over the segment's rows as colsum_tile_kernel does
// (every row of a row lane's share loaded before the first add), writes the
// partials with device-scope stores, waits for them, and counts itself in on
// its chunk's counter; the chunk's last block adds the chunk's partials in
// segment order (256 / (16 W) threads per column, each a contiguous range of
// segments, their sums then added in range order), writes the float sums and
// resets the counter for the next launch (launches on the library's stream
// never overlap). The result does not depend on which block is last.
constexpr int kMaxFinishChunks = 1 << 16;
__device__ unsigned int g_colsum_done[kMaxFinishChunks];

template <bool Vec, int Block>
__global__ __launch_bounds__(Block) void colsum_finish_kernel(const float* __restrict__ x, double* __restrict__ part,
                                                              float* __restrict__ out, int64_t len, int64_t inner,
                                                              int64_t seg_len) {
    constexpr int W = Vec ? 4 : 1;
    constexpr int kWaves = Block / kWave;
    constexpr int kRows = Block / kColLanes;  // row lanes of a block
    constexpr int kCols = kColLanes * W;      // columns of a block
    constexpr int kParts = Block / kCols;     // threads per column in the final sum
    __shared__ double lds[kWaves][kCols];
    __shared__ int last_block;
    const int c = threadIdx.x % kColLanes, rl = threadIdx.x / kColLanes;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    // Workgroups go to the 8 XCDs round robin by linear id. When a row is not
    // whole 128-byte lines, neighbouring chunks share lines at their edges:
    // each XCD then takes a contiguous run of chunks, so that most shared
    // lines are fetched into one XCD's L2 (8192 x 1000: 39 MB fetched instead
    // of 46 MB, 11.3 us instead of 12.3 us). Rows of whole lines keep the
    // plain order: remapped, 8192 x 4096 took 26.2 us instead of 24.2 us.
    int64_t chunk = blockIdx.x, s = blockIdx.y;
    const int64_t segs = gridDim.y, nchunks = gridDim.x;
    if (nchunks % 8 == 0 && (inner * int64_t(sizeof(float))) % 128 != 0) {
        const int64_t linear = int64_t(blockIdx.x) + int64_t(blockIdx.y) * nchunks;
        const int64_t per = nchunks / 8, j = linear / 8;
        chunk = (linear % 8) * per + j % per;
        s = j / per;
    }
    const int64_t col = (chunk * kColLanes + c) * W;
    const int64_t a0 = s * seg_len, a1 = std::min(len, a0 + seg_len);
    double acc[W];
#pragma unroll
    for (int w = 0; w < W; ++w) acc[w] = 0.0;
    if (col < inner) {
        const float* base = x + col;
        for (int64_t a = a0 + rl; a < a1; a += kColInFlight * kRows) {
            // Up to kColInFlight rows, all loaded before the first add.
            if constexpr (Vec) {
                f4 v[kColInFlight];
#pragma unroll
                for (int u = 0; u < kColInFlight; ++u) {
                    const int64_t r = a + u * kRows;
                    v[u] = r < a1 ? ld4(base + r * inner) : f4{0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
                for (int u = 0; u < kColInFlight; ++u) {
                    if (a + u * kRows < a1) {
                        acc[0] += double(v[u].x); acc[1] += double(v[u].y); acc[2] += double(v[u].z); acc[3] += double(v[u].w);
                    }
                }
            } else {
                float v[kColInFlight];
#pragma unroll
                for (int u = 0; u < kColInFlight; ++u) {
                    const int64_t r = a + u * kRows;
                    v[u] = r < a1 ? base[r * inner] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < kColInFlight; ++u)
                    if (a + u * kRows < a1) acc[0] += double(v[u]);
            }
        }
    }
#pragma unroll
    for (int w = 0; w < W; ++w) {
        acc[w] += __shfl_xor(acc[w], 16, kWave);
        acc[w] += __shfl_xor(acc[w], 32, kWave);
    }
    if (lane < kColLanes) {
#pragma unroll
        for (int w = 0; w < W; ++w) lds[wave][c * W + w] = acc[w];
    }
    __syncthreads();
    if (wave == 0 && lane < kColLanes) {
#pragma unroll
        for (int w = 0; w < W; ++w) {
            double total = lds[0][c * W + w];
#pragma unroll
            for (int k = 1; k < kWaves; ++k) total += lds[k][c * W + w];
            if (col + w < inner)
                __hip_atomic_store(&part[s * inner + col + w], total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // A device-scope store is acknowledged once it is visible at device
        // scope: waiting for every outstanding memory operation orders these
        // stores before the count below.
        red::wait_stores_visible();
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned* counter = &g_colsum_done[chunk];
        const bool last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 ==
                          unsigned(segs);
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_block = last;
    }
    __syncthreads();
    if (!last_block) return;
    // Thread t: column t % kCols of the chunk, segments of range t / kCols.
    const int cc = int(threadIdx.x) % kCols, q = int(threadIdx.x) / kCols;
    const int64_t ocol = chunk * kCols + cc;
    const int64_t per = (segs + kParts - 1) / kParts;
    const int64_t s0 = std::min<int64_t>(segs, q * per), s1 = std::min<int64_t>(segs, s0 + per);
    // Device-scope loads (cache policy sc1 = 16), eight in flight; a load
    // past the partials falls outside the descriptor and reads 0 (not added).
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        part, short(0), int(std::min<int64_t>(segs * inner * int64_t(sizeof(double)), 0x7fffffff)), 0x00020000);
    double sum = 0.0;
    if (ocol < inner) {
        for (int64_t t0 = s0; t0 < s1; t0 += 8) {
            double v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t t = t0 + u;
                const int64_t off = t < s1 ? (t * inner + ocol) * int64_t(sizeof(double)) : int64_t(0x7fffffff);
                v[u] = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(rp, int(off), 0, 16));
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (t0 + u < s1) sum += v[u];
        }
    }
    __shared__ double range_sum[kParts][kCols];
    range_sum[q][cc] = sum;
    __syncthreads();
    if (q == 0 && ocol < inner) {
        double total = range_sum[0][cc];
        for (int k = 1; k < kParts; ++k) total += range_sum[k][cc];
        out[ocol] = float(total);
    }
}

// out[t] = float(sum over segments of part[s][t]), in segment order. All
// segments' loads are issued before the first add (one memory round trip).
constexpr int kMaxColSegs = 64;
__global__ __launch_bounds__(kBlock) void colsum_combine_kernel(const double* __restrict__ part, float* __restrict__ out,
                                                                int64_t total, int segs) {
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    double v[kMaxColSegs];
#pragma unroll
    for (int s = 0; s < kMaxColSegs; ++s)
        if (s < segs) v[s] = part[s * total + t];
    double acc = 0.0;
#pragma unroll
    for (int s = 0; s < kMaxColSegs; ++s)
        if (s < segs) acc += v[s];
    out[t] = float(acc);
}

// ---- split columns for max/argmax --------------------------------------------------
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

// Segments of a column sum: a function of the shape only; aim at ~512
// long-running workgroups (two per CU), at least 128 rows per segment, at
// most 64 segments. A reduction of at most 2^17 elements takes one segment
// and one launch: its time is the launches', not the bytes'.
struct ColumnPlan {
    bool vec;
    int64_t chunks, segs, seg_len;
};

ColumnPlan column_plan(const float* in, int64_t outer, int64_t len, int64_t inner) {
    ColumnPlan c{};
    c.vec = inner % 4 == 0 && aligned16(in);
    const int64_t width = c.vec ? 4 * kColLanes : kColLanes;
    c.chunks = (inner + width - 1) / width;
    const int64_t blocks_x = outer * c.chunks;
    if (blocks_x > std::numeric_limits<int>::max()) fail(VC_HIP_ERR_OVERFLOW, "reduction too large");
    int64_t segs = std::max<int64_t>(1, (512 + blocks_x - 1) / blocks_x);
    segs = std::min<int64_t>({segs, std::max<int64_t>(1, len / 128), int64_t(kMaxColSegs)});
    if (outer * len * inner <= (int64_t(1) << 17)) segs = 1;
    c.seg_len = (len + segs - 1) / segs;
    c.segs = (len + c.seg_len - 1) / c.seg_len;
    return c;
}

// The one-launch column sum (outer 1): about 2048 blocks from 32 chunks
// (2048 columns) up, about 128 from 8 to 31 chunks; segments of at least 256
// rows, at most 32 segments (the blocks of a chunk count in on one counter,
// and atomics on one address are served one at a time: 128 segments per chunk
// measured 2.5x slower than 32); a function of the shape only. Narrow sums
// take few, long segments: with 512 blocks their counters queued and
// 8192 x 1000 took 13.9 us, against 12.1-12.4 us for 128 blocks and for the
// two-launch path, which 4096 x 1000 takes in 8.9 us against 7.3 us here.
// Below 8 chunks the two-launch path runs. (8192 x 4096 takes 23.9 us in one
// launch against 26.1 us in two.) Narrow sums run 512-thread workgroups, twice
// the rows in flight per block at the same count of partials and counters:
// 8192 x 1000 11.5 -> 10.2 us, 4096 x 1000 7.3 -> 7.0 us, 8192 x 512 the
// same 7.0 us; 1024 threads gave 10.3 us on 8192 x 1000 but 7.8 and 8.0 us on
// the other two, and 256 blocks of 512 threads 11.1 us (back-to-back calls).
// Wide sums keep 256 threads: 512 or 1024 at 1024-2048 blocks measured the
// same or slower (1024 threads at 2048 blocks: 39 us on 8192 x 4096).
#ifndef VC_COLSUM_NARROW_BLOCK
#define VC_COLSUM_NARROW_BLOCK 512
#endif
#ifndef VC_COLSUM_NARROW_BLOCKS
#define VC_COLSUM_NARROW_BLOCKS 128
#endif
#ifndef VC_COLSUM_WIDE_BLOCK
#define VC_COLSUM_WIDE_BLOCK 256
#endif
#ifndef VC_COLSUM_WIDE_BLOCKS
#define VC_COLSUM_WIDE_BLOCKS 2048
#endif
// Segments shorter than 256 rows cost more in partials and counter atomics
// than they give in parallel loads: with the floor at 16 rows, 1024 x 4096
// ran as 32 segments of 32 rows in 14.6 us; at 256 rows, 4 segments take
// 6.2-6.4 us (512 x 4096 14.5 -> 5.7, 2048 x 2048 10.6 -> 6.5, 256 x 8192
// 10.0 -> 5.4 us). A floor of 512 rows lost 23% on 1000 x 4096 (two
// segments), 1024 lost on most shapes. The step's shapes keep their plans.
#ifndef VC_COLSUM_MIN_SEG_ROWS
#define VC_COLSUM_MIN_SEG_ROWS 256
#endif
constexpr int64_t kFinishMinChunks = 8, kFinishWideChunks = 32;
struct FinishPlan {
    bool vec;
    int block;  // threads per workgroup: 256, 512 or 1024
    int64_t chunks, segs, seg_len;
};

FinishPlan finish_plan(const float* in, int64_t len, int64_t inner) {
    FinishPlan f{};
    f.vec = inner % 4 == 0 && aligned16(in);
    const int64_t width = f.vec ? 4 * kColLanes : kColLanes;
    f.chunks = (inner + width - 1) / width;
    const bool wide = f.chunks >= kFinishWideChunks;
    f.block = wide ? VC_COLSUM_WIDE_BLOCK : VC_COLSUM_NARROW_BLOCK;
    const int64_t blocks = wide ? VC_COLSUM_WIDE_BLOCKS : VC_COLSUM_NARROW_BLOCKS;
    int64_t segs = std::max<int64_t>(1, (blocks + f.chunks - 1) / f.chunks);
    segs = std::min<int64_t>({segs, std::max<int64_t>(1, len / VC_COLSUM_MIN_SEG_ROWS), int64_t(32)});
    f.seg_len = (len + segs - 1) / segs;
    f.segs = (len + f.seg_len - 1) / f.seg_len;
    return f;
}

void column_sum(Device& d, const ColumnPlan& c, const float* in, float* out, double* part, int64_t outer,
                int64_t len, int64_t inner, const char* label) {
    const int64_t total = outer * inner;
    const dim3 grid(static_cast<unsigned>(outer * c.chunks), static_cast<unsigned>(c.segs));
    if (c.segs == 1) {
        if (c.vec)
            launch(colsum_tile_kernel<true, true>, grid, dim3(kBlock), 0, d.stream, in, part, out, outer, len, inner,
                   c.seg_len, c.chunks);
        else
            launch(colsum_tile_kernel<false, true>, grid, dim3(kBlock), 0, d.stream, in, part, out, outer, len, inner,
                   c.seg_len, c.chunks);
        after_launch(label);
        return;
    }
    if (c.vec)
        launch(colsum_tile_kernel<true, false>, grid, dim3(kBlock), 0, d.stream, in, part, out, outer, len, inner,
               c.seg_len, c.chunks);
    else
        launch(colsum_tile_kernel<false, false>, grid, dim3(kBlock), 0, d.stream, in, part, out, outer, len, inner,
               c.seg_len, c.chunks);
    after_launch(label);
    launch(colsum_combine_kernel, dim3(unsigned((total + kBlock - 1) / kBlock)), dim3(kBlock), 0, d.stream, part, out,
           total, int(c.segs));
    after_launch(label);
}

// Segments of a max/argmax over a long axis with few outputs (>= 16 rows each).
struct BestPlan {
    int64_t segs, seg_len;
};

BestPlan best_plan(int64_t len, int64_t total, int64_t target_threads) {
    BestPlan b{};
    int64_t segs = std::min<int64_t>((target_threads + total - 1) / total, (len + 15) / 16);
    segs = std::max<int64_t>(1, std::min<int64_t>(segs, 1024));
    b.seg_len = (len + segs - 1) / segs;
    b.segs = (len + b.seg_len - 1) / b.seg_len;
    return b;
}

// Device memory for one call's partial results: pool buffers
// (vc_hip_reduce_axis) or the static array (vc_hip_reduce_axis_noalloc).
class PartialMemory {
public:
    virtual ~PartialMemory() = default;
    virtual void* take(size_t bytes) = 0;
};

class PoolPartials final : public PartialMemory {
public:
    void* take(size_t bytes) override {
        held_.push_back(std::make_unique<Scratch>(bytes));
        return held_.back()->as<void>();
    }

private:
    std::vector<std::unique_ptr<Scratch>> held_;
};

void reduce_axis(const float* in, float* out, int64_t outer, int64_t len, int64_t inner, int op,
                 PartialMemory& memory) {
    Device& d = require_device();
    if (op < VC_REDUCE_SUM || op > VC_REDUCE_ARGMAX) fail(VC_HIP_ERR_INVALID_ARGUMENT, "unknown reduction");
    if (len == 0 && op != VC_REDUCE_SUM) fail(VC_HIP_ERR_INVALID_ARGUMENT, "max/argmax over an empty axis is undefined");
    const int64_t total = outer * inner;
    if (total == 0) return;
    const char* label = op == VC_REDUCE_SUM ? "reduce_axis_sum" : op == VC_REDUCE_MAX ? "reduce_axis_max" : "reduce_axis_argmax";
    if (len == 0) {  // sum over an empty axis is zero
        launch(zero_kernel, dim3(grid_1d(size_t(total), kBlock, 1024)), dim3(kBlock), 0, d.stream, out, total);
        after_launch(label);
        return;
    }
    check_i32(len, "reduction axis length");
    Profiled p(label, double(outer * len * inner), 4.0 * double(outer * len * inner + total));
    const int64_t target_threads = int64_t(d.cu_count) * 1024;
    if (inner == 1) {
        // One wavefront per row; rows of < 64 elements leave lanes idle but stay correct.
        const bool vec = len % 4 == 0 && aligned16(in);
        const unsigned grid = unsigned(std::min<int64_t>((outer + 3) / 4, int64_t(d.cu_count) * 64));
        const int64_t nv = vec ? (len + kWave * 4 - 1) / (kWave * 4) : 0;
#define VC_ROWS_NV(OP, VEC, NV) \
    launch((rows_kernel<OP, VEC, NV>), dim3(grid), dim3(kBlock), 0, d.stream, in, out, outer, len)
#define VC_ROWS(OP)                                 \
    if (!vec) VC_ROWS_NV(OP, false, 0);             \
    else if (nv <= 1) VC_ROWS_NV(OP, true, 1);      \
    else if (nv <= 2) VC_ROWS_NV(OP, true, 2);      \
    else if (nv <= 4) VC_ROWS_NV(OP, true, 4);      \
    else if (nv <= 8) VC_ROWS_NV(OP, true, 8);      \
    else if (nv <= 16) VC_ROWS_NV(OP, true, 16);    \
    else VC_ROWS_NV(OP, true, 0)
        if (op == VC_REDUCE_SUM) { VC_ROWS(0); }
        else if (op == VC_REDUCE_MAX) { VC_ROWS(1); }
        else { VC_ROWS(2); }
#undef VC_ROWS
#undef VC_ROWS_NV
        after_launch(label);
        p.done();
        return;
    }
    if (total >= target_threads || len < 64) {
        const unsigned grid = grid_1d(size_t(total), kBlock, unsigned(d.cu_count) * 64);
        if (op == VC_REDUCE_SUM) launch(cols_kernel<0>, dim3(grid), dim3(kBlock), 0, d.stream, in, out, outer, len, inner);
        else if (op == VC_REDUCE_MAX) launch(cols_kernel<1>, dim3(grid), dim3(kBlock), 0, d.stream, in, out, outer, len, inner);
        else launch(cols_kernel<2>, dim3(grid), dim3(kBlock), 0, d.stream, in, out, outer, len, inner);
        after_launch(label);
        p.done();
        return;
    }
    if (op == VC_REDUCE_SUM && outer == 1 && len * inner > (int64_t(1) << 17)) {
        const FinishPlan f = finish_plan(in, len, inner);
        const int64_t part_bytes = f.segs * inner * int64_t(sizeof(double));
        if (f.chunks >= kFinishMinChunks && f.chunks <= kMaxFinishChunks && part_bytes < (int64_t(1) << 31)) {
            double* part = static_cast<double*>(memory.take(size_t(part_bytes)));
            const dim3 grid(unsigned(f.chunks), unsigned(f.segs));
#define VC_FINISH(VEC, B) \
    launch(colsum_finish_kernel<VEC, B>, grid, dim3(B), 0, d.stream, in, part, out, len, inner, f.seg_len)
            if (f.block == 1024) {
                if (f.vec) VC_FINISH(true, 1024); else VC_FINISH(false, 1024);
            } else if (f.block == 512) {
                if (f.vec) VC_FINISH(true, 512); else VC_FINISH(false, 512);
            } else {
                if (f.vec) VC_FINISH(true, 256); else VC_FINISH(false, 256);
            }
#undef VC_FINISH
            after_launch(label);
            p.done();
            return;
        }
    }
    if (op == VC_REDUCE_SUM) {
        const ColumnPlan c = column_plan(in, outer, len, inner);
        // One segment: colsum_tile_kernel writes the sums directly and never
        // touches partials, so none are taken.
        double* part =
            c.segs > 1 ? static_cast<double*>(memory.take(size_t(c.segs * total) * sizeof(double))) : nullptr;
        column_sum(d, c, in, out, part, outer, len, inner, label);
        p.done();
        return;
    }
    // max/argmax with few outputs: split the axis into segments.
    const BestPlan b = best_plan(len, total, target_threads);
    const dim3 grid1(unsigned((total + kBlock - 1) / kBlock), unsigned(b.segs));
    const unsigned grid2 = unsigned((total + kBlock - 1) / kBlock);
    char* mem = static_cast<char*>(memory.take(size_t(b.segs * total) * (sizeof(float) + sizeof(int))));
    float* pv = reinterpret_cast<float*>(mem);
    int* pi = reinterpret_cast<int*>(mem + size_t(b.segs * total) * sizeof(float));
    launch(cols_best_partial_kernel, grid1, dim3(kBlock), 0, d.stream, in, pv, pi, outer, len, inner, b.seg_len);
    after_launch(label);
    if (op == VC_REDUCE_MAX)
        launch(cols_best_combine_kernel<1>, dim3(grid2), dim3(kBlock), 0, d.stream, in, pv, pi, out, outer, len, inner,
               b.segs);
    else
        launch(cols_best_combine_kernel<2>, dim3(grid2), dim3(kBlock), 0, d.stream, in, pv, pi, out, outer, len, inner,
               b.segs);
    after_launch(label);
    p.done();
}

// ---- partial results without allocation (vc_hip_reduce_axis_noalloc) ------------
// A file-scope device array holds the partial results of the
// allocation-free entry point; each GPU that loads the library holds its own
// copy until the process ends. On the host, `scratch` names a stand-in, not
// device memory: host code uses only the address that hipGetSymbolAddress
// returns for the current device. A column sum keeps segs * outputs at most
// 2048 * 64 + outputs double partials (one launch; 512 * 64 + outputs with a
// separate combine), so 2 MiB holds the column sums of up to 2^17 outputs:
// the bias gradient of a [8192, 4096] layer needs 1 MiB (32 segments). A
// max/argmax split over a long axis with few outputs needs 8 bytes per
// (segment, output); a shape that needs more than the array is rejected.
constexpr size_t kNoAllocScratchBytes = size_t(2) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

// The address of this device's copy of `scratch`, resolved once per device
// with that device current.
void* noalloc_scratch(const Device& d) {
    static std::mutex mu;
    static void* address[kMaxDevices] = {};
    if (d.ordinal < 0 || d.ordinal >= kMaxDevices) fail(VC_HIP_ERR_RUNTIME, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (!address[d.ordinal]) {
        void* p = nullptr;
        check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress (reduction scratch)");
        if (!p) fail(VC_HIP_ERR_RUNTIME, "hipGetSymbolAddress returned no address for the reduction scratch");
        address[d.ordinal] = p;
    }
    return address[d.ordinal];
}

// Hands out 256-byte-aligned pieces of the static array, in order; fails,
// before anything is launched, when a call needs more than it holds.
class StaticPartials final : public PartialMemory {
public:
    explicit StaticPartials(void* base) : base_(static_cast<char*>(base)) {}
    void* take(size_t bytes) override {
        const size_t begin = (used_ + 255) / 256 * 256;
        if (bytes > kNoAllocScratchBytes || begin > kNoAllocScratchBytes - bytes)
            fail(VC_HIP_ERR_INVALID_ARGUMENT,
                 "vc_hip_reduce_axis_noalloc: this reduction needs " + std::to_string(begin + bytes) +
                     " bytes of partial results; the allocation-free entry point holds " +
                     std::to_string(kNoAllocScratchBytes) + " (use vc_hip_reduce_axis)");
        used_ = begin + bytes;
        return base_ + begin;
    }

private:
    char* base_;
    size_t used_ = 0;
};

}  // namespace

void ColsumRelease::operator()(vc_hip_colsum* h) const noexcept {
    if (!h) return;
    pool_release(h->part);
    delete h;
}

ColsumPtr new_colsum(int64_t rows, int64_t n) {
    if (rows <= 0 || n <= 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "pending column sums need at least one row and column");
    void* part = pool_alloc(size_t(rows) * size_t(n) * sizeof(double));
    return ColsumPtr(new vc_hip_colsum{static_cast<double*>(part), rows, n});
}

void finish_colsum(const vc_hip_colsum& h, float* out) {
    Device& d = require_device();
    Profiled p("column_sum_combine", 0.0, 8.0 * double(h.rows * h.n) + 4.0 * double(h.n));
    launch(red::column_partials_kernel, dim3(unsigned((h.n + 63) / 64)), dim3(64 * red::kCombineWaves), 0, d.stream,
           static_cast<const double*>(h.part), h.rows, h.n, out);
    after_launch("column_sum_combine");
    p.done();
}

}  // namespace vchip

using namespace vchip;

extern "C" {

int vc_hip_reduce_sum(const float* in, size_t count, float* out) {
    return guard([&] {
        Device& d = require_device();
        if (!out) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_reduce_sum: null output");
        const int64_t n = int64_t(count);
        const int64_t chunk = red::sum_chunk(n);
        // One launch: at most 2048 chunks (sum_chunk), at least one block.
        const int64_t blocks = std::max<int64_t>(1, (n + chunk - 1) / chunk);
        Scratch part(size_t(blocks) * sizeof(double));
        Profiled p("reduce_sum", double(n), 4.0 * double(n));
        if (aligned16(in))
            launch(red::sum_finish_kernel<true, red::Identity>, dim3(unsigned(blocks)), dim3(kBlock), 0, d.stream, in,
                   part.as<double>(), out, n, chunk, red::Identity());
        else
            launch(red::sum_finish_kernel<false, red::Identity>, dim3(unsigned(blocks)), dim3(kBlock), 0, d.stream,
                   in, part.as<double>(), out, n, chunk, red::Identity());
        after_launch("reduce_sum");
        p.done();
    });
}

int vc_hip_reduce_axis(const float* in, float* out, size_t outer, size_t length, size_t inner, int op) {
    return guard([&] {
        PoolPartials memory;
        reduce_axis(in, out, int64_t(outer), int64_t(length), int64_t(inner), op, memory);
    });
}

int vc_hip_reduce_axis_noalloc(const float* in, float* out, size_t outer, size_t length, size_t inner, int op) {
    return guard([&] {
        Device& d = require_device();
        // One call at a time fills the array and enqueues the kernels that
        // read it; the library's single in-order stream then runs calls one
        // after another, so a call never sees another's partial results.
        static std::mutex serial;
        std::lock_guard<std::mutex> lock(serial);
        StaticPartials memory(noalloc_scratch(d));
        reduce_axis(in, out, int64_t(outer), int64_t(length), int64_t(inner), op, memory);
    });
}

int vc_hip_scatter_axis(const float* values, const float* indices, float* out, size_t outer, size_t length, size_t inner) {
    return guard([&] {
        Device& d = require_device();
        const int64_t total = int64_t(outer * length * inner);
        if (total == 0) return;
        Profiled p("scatter_axis", 0.0, 4.0 * double(total + 2 * outer * inner));
        launch(scatter_kernel, dim3(grid_1d(size_t(total), kBlock, unsigned(d.cu_count) * 16)), dim3(kBlock), 0,
                           d.stream, values, indices, out, int64_t(outer), int64_t(length), int64_t(inner));
        after_launch("scatter_axis");
        p.done();
    });
}

int vc_hip_transpose_last2(const float* in, float* out, size_t batch, size_t rows, size_t cols) {
    return guard([&] {
        Device& d = require_device();
        if (batch * rows * cols == 0) return;
        if ((rows + kTile - 1) / kTile > 65535) fail(VC_HIP_ERR_OVERFLOW, "transpose: too many rows");
        const dim3 grid(unsigned((cols + kTile - 1) / kTile), unsigned((rows + kTile - 1) / kTile),
                        unsigned(std::min<size_t>(batch, 65535)));
        Profiled p("transpose_last2", 0.0, 8.0 * double(batch * rows * cols));
        launch(transpose_kernel, grid, dim3(kTile, 8), 0, d.stream, in, out, int64_t(batch), int64_t(rows),
                           int64_t(cols));
        after_launch("transpose_last2");
        p.done();
    });
}

int vc_hip_colsum_finish(const vc_hip_colsum* sums, float* column_sum) {
    return guard([&] {
        if (!sums || !column_sum) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_colsum_finish: null pointer");
        finish_colsum(*sums, column_sum);
    });
}

int vc_hip_colsum_size(const vc_hip_colsum* sums, size_t* columns) {
    return guard([&] {
        if (!sums || !columns) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_colsum_size: null pointer");
        *columns = size_t(sums->n);
    });
}

int vc_hip_colsum_release(vc_hip_colsum* sums) {
    return guard([&] { ColsumRelease()(sums); });
}

}  // extern "C"
